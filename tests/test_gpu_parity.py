"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Mirrors the reference's integration suite (tests/correctness.rs) and its
differential fuzzer (fuzz/fuzz_targets/flash_attention.rs), with the bar
tightened to north_star's: max-abs < 2e-5 and relative L2 < 1e-5 against the
oracle's CPU v2 (oracle/fa_oracle.c, restating src/v2.rs:160-385) on the same
inputs.  The oracle itself is pinned by tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import flash_attention_amd as fa
import oracle
from fa_testutil import (NAIVE_TOL, assert_parity, attention_f64, max_abs_diff, normal_vec, random_vec,
                         rel_l2, uniform_vec)

pytestmark = pytest.mark.gpu

ALL_VARIANTS = (1, 2, 3)


@pytest.fixture(scope="module", autouse=True)
def _device():
    fa.init()   # raises FaError without a device / code object: no silent fallback


def cpu_v2(q, k, v, bh, sq, sk, d, causal):
    return oracle.run(2, q, k, v, bh, sq, sk, d, causal, 64, 128)


def run_case(variant, seq_q, seq_k, d, br, bc, causal):
    """tests/correctness.rs:73-113 with the GPU as the flash implementation."""
    q = random_vec(seq_q * d, 1)
    k = random_vec(seq_k * d, 2)
    v = random_vec(seq_k * d, 3)
    out = np.zeros(seq_q * d, dtype=np.float32)
    cfg = fa.FlashAttentionConfig(br, bc, causal)
    fa.VARIANTS[variant](q, k, v, seq_q, seq_k, d, cfg, out)
    what = f"v{variant} seq_q={seq_q} seq_k={seq_k} d={d} br={br} bc={bc} causal={causal}"
    naive = oracle.naive_f64(q, k, v, seq_q, seq_k, d, causal)
    assert max_abs_diff(out, naive) < NAIVE_TOL, what
    assert_parity(out, cpu_v2(q, k, v, 1, seq_q, seq_k, d, causal), what)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_matches_exact_block_multiples(variant):
    run_case(variant, 64, 64, 64, 32, 32, False)
    run_case(variant, 128, 128, 64, 64, 64, False)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_matches_ragged_sizes(variant):
    for case in [(17, 23, 32, 8, 8), (1, 1, 16, 8, 8), (1, 50, 33, 16, 16), (50, 1, 33, 16, 16),
                 (97, 131, 17, 32, 40), (200, 200, 128, 64, 128)]:
        run_case(variant, *case, False)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_block_sizes_not_multiple_of_four(variant):
    for b in (3, 5, 6, 7):
        for causal in (False, True):
            run_case(variant, 23, 29, 24, b, 12, causal)
            run_case(variant, 29, 23, 24, 12, b, causal)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_matches_causal(variant):
    run_case(variant, 64, 64, 64, 32, 32, True)
    run_case(variant, 97, 97, 33, 16, 24, True)
    run_case(variant, 1, 1, 16, 8, 8, True)
    run_case(variant, 5, 5, 8, 64, 64, True)
    run_case(variant, 10, 40, 32, 4, 8, True)   # asymmetric, top-left aligned
    run_case(variant, 10, 10, 8, 1024, 1024, False)
    run_case(variant, 10, 10, 8, 1024, 1024, True)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_every_padded_head_dim(variant):
    # d_head 1..256 across the 32/64/128/256 kernels, both load paths.
    for d in (1, 2, 3, 4, 5, 8, 16, 31, 32, 40, 48, 63, 64, 65, 96, 127, 128, 129, 160, 200, 255, 256):
        run_case(variant, 70, 90, d, 64, 128, d % 2 == 0)


def _wide_kernel(d):
    return 512 if d <= 512 else (1024 if d <= 1024 else 2048)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_wide_heads_run_flash_kernels(variant):
    # The crate's flash path takes any d_head with O(block) scratch
    # (src/v2.rs:182-189): heads of 257..2048 columns run the column-group
    # flash kernels (no score matrix), odd widths on the scalar loader.
    for d in (257, 300, 384, 512, 513, 640, 1000, 1023, 1024, 1025, 1536, 2047, 2048):
        plan = fa.describe_launch(variant, 1, 1, 70, 90, d, d % 2 == 1)
        assert plan.startswith(f"fa_prefill_v{variant}_d{_wide_kernel(d)}_"), plan
        run_case(variant, 70, 90, d, 64, 128, d % 2 == 1)
    bh, sq, sk, d = 3, 65, 129, 320
    q, k, v = random_vec(bh * sq * d, 4), random_vec(bh * sk * d, 5), random_vec(bh * sk * d, 6)
    want = cpu_v2(q, k, v, bh, sq, sk, d, True)
    out = np.zeros(bh * sq * d, np.float32)
    fa.MULTIHEAD_VARIANTS[variant](q, k, v, 1, bh, sq, sk, d, fa.FlashAttentionConfig(causal=True), out)
    assert_parity(out, want, f"v{variant} multihead d={d}")
    assert_parity(_device_run(variant, q, k, v, bh, sq, sk, d, True, guard=64), want, f"v{variant} device d={d}")
    # explicit scale: attention with scale s equals default attention on Q * (s * sqrt(d))
    scale = 0.03
    q2 = (q.astype(np.float64) * scale * np.sqrt(d)).astype(np.float32)
    want2 = np.concatenate([attention_f64(q2[h * sq * d:(h + 1) * sq * d], k[h * sk * d:(h + 1) * sk * d],
                                          v[h * sk * d:(h + 1) * sk * d], sq, sk, d, True) for h in range(bh)])
    assert max_abs_diff(_device_run(variant, q, k, v, bh, sq, sk, d, True, scale=scale), want2) < 1e-5


def test_v1_rows_past_their_causal_end_do_not_drift():
    """v1 visits every key stage (no causal skip, src/v1.rs:209-216), so a
    causal row whose visible keys end early meets many stages that add
    nothing; those skip the un-normalise / re-normalise round trip (an
    identity whose o * l * fl(1/l) would move o by an ulp-scale step per
    stage).  Few queries over many keys is the worst case: rows see <= sq keys
    and then hundreds of empty stages (found by a random differential run:
    4 x 24 x 5671, d 256, max-abs 2.1e-5 before)."""
    rng = np.random.default_rng(2024)
    for bh, sq, sk, d in ((4, 24, 5671, 256), (2, 64, 8192, 128), (1, 40, 3000, 512), (3, 16, 4000, 64)):
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, True)
        tag = f"v1 ({bh},{sq},{sk},{d}) causal: {fa.describe_launch(1, 1, bh, sq, sk, d, True)}"
        print("[case]", tag, flush=True)
        got = _device_run(1, q, k, v, bh, sq, sk, d, True, guard=64)
        assert_parity(got, want, tag)
        # as close to v2 as v2's own kernel is (no per-stage drift left)
        v2 = _device_run(2, q, k, v, bh, sq, sk, d, True)
        assert max_abs_diff(got, want) < 2.0 * max_abs_diff(v2, want) + 2e-6, tag


@pytest.mark.parametrize("d", (384, 512, 1024))
def test_wide_heads_multiblock_and_key_split(d):
    """Several query blocks with causal skipping, ragged ends, and the key
    split (automatic and forced) at wide heads; every variant against CPU v2,
    v1 / v2 / v3 against each other."""
    rng = np.random.default_rng(d)
    for bh, sq, sk, causal in [(2, 300, 300, True), (1, 130, 700, False), (5, 77, 77, True)]:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        outs = {}
        for variant in ALL_VARIANTS:
            outs[variant] = _device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=64)
            assert_parity(outs[variant], want, f"v{variant} {bh},{sq},{sk},{d},{causal}")
        assert_parity(outs[1], outs[2], "v1 vs v2")
        assert_parity(outs[3], outs[2], "v3 vs v2")
        for variant in ALL_VARIANTS:
            for splits in (2, 3, 5):
                plan = fa.describe_launch(variant, 1, bh, sq, sk, d, causal, fa.PATH_PREFILL, splits)
                out = _device_run(variant, q, k, v, bh, sq, sk, d, causal, fa.PATH_PREFILL, splits, guard=64)
                assert_parity(out, want, f"v{variant} split {splits}: {plan}")


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_heads_of_1025_to_2048_columns_run_flash_kernels(variant):
    """d = 1025, 1536, 2048 (the crate's flash path at any d_head,
    src/v2.rs:182-189): the D = 2048 kernels -- 16-row workgroups of 8
    column-group waves, K and V in turn through one LDS buffer -- with no
    score buffer in the plan; several query blocks, causal and ragged, the key
    split (automatic on small grids, and forced) and the stream split, every
    variant against CPU v2 and against each other."""
    rng = np.random.default_rng(2048 + variant)
    for bh, sq, sk, d, causal in [(2, 100, 130, 1025, True), (1, 37, 300, 1536, False), (3, 64, 64, 2048, True),
                                  (1, 200, 90, 2048, False)]:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for path, splits in ((fa.PATH_AUTO, 0), (fa.PATH_PREFILL, 0), (fa.PATH_PREFILL, 3), (fa.PATH_STREAM, 5)):
            plan = fa.describe_launch(variant, 1, bh, sq, sk, d, causal, path, splits)
            assert plan.startswith(f"fa_prefill_v{variant}_d2048_") and "naive" not in plan, plan
            tag = f"v{variant} ({bh},{sq},{sk},{d},{causal}) {plan}"
            print("[case]", tag, flush=True)
            assert_parity(_device_run(variant, q, k, v, bh, sq, sk, d, causal, path, splits, guard=64), want, tag)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_heads_wider_than_2048_run_flash_kernels(variant):
    """d > 2048 (the crate's flash path at any d_head, src/v2.rs:175-189):
    the any-width kernels -- one workgroup per 16-row tile, O accumulated in
    registers up to 4096 columns, in the output rows beyond -- with no score
    buffer and no workspace.  Widths with a ragged last 64-column chunk and
    with d % 4 != 0 (scalar loads), ragged query tiles, key ends inside a
    64-key stage, causal with seq_q < seq_k and > seq_k, several slices,
    waves with fewer chunks than others; every variant against CPU v2 and the
    f64 naive oracle; forced prefill path as the automatic one."""
    rng = np.random.default_rng(4096 + variant)
    for bh, sq, sk, d, causal in [(1, 20, 30, 2049, True), (1, 33, 17, 2100, False), (2, 40, 100, 3000, True),
                                  (1, 70, 45, 4096, True), (2, 17, 130, 2052, False), (1, 30, 70, 4097, True),
                                  (1, 19, 50, 5000, False)]:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for path in (fa.PATH_AUTO, fa.PATH_PREFILL):
            plan = fa.describe_launch(variant, 1, bh, sq, sk, d, causal, path)
            kind = "dreg" if d <= 4096 else "dany"
            assert plan.startswith(f"fa_prefill_v{variant}_{kind}_{1 if d % 4 == 0 else 0} ") and \
                "workspace" not in plan, plan
            tag = f"v{variant} ({bh},{sq},{sk},{d},{causal}) {plan}"
            print("[case]", tag, flush=True)
            got = _device_run(variant, q, k, v, bh, sq, sk, d, causal, path, 0, guard=64)
            assert_parity(got, want, tag)
        for h in range(bh):
            sl_q = slice(h * sq * d, (h + 1) * sq * d)
            sl_k = slice(h * sk * d, (h + 1) * sk * d)
            naive = oracle.naive_f64(q[sl_q], k[sl_k], v[sl_k], sq, sk, d, causal)
            assert max_abs_diff(got[sl_q], naive) < NAIVE_TOL, tag
    # the host-slice entry point takes the same kernels
    run_case(variant, 20, 30, 2049, 64, 128, True)


def test_heads_wider_than_2048_differential_fuzz():
    """Random shapes on the any-width kernels: d_head 2049..6000 (O in
    registers up to 4096 columns, in the output rows beyond; scalar loads
    when d % 4 != 0), 1..4 slices, ragged query and key counts (a query tile
    or 64-key stage cut anywhere), causal or not, logits up to sigma 2;
    v1 / v2 / v3 against CPU v2, and v2 / v3 bit-identical (v3 runs v2's
    steps on these kernels)."""
    rng = np.random.default_rng(6000)
    for case in range(8):
        d = int(rng.integers(2049, 6001))
        bh = int(rng.integers(1, 5))
        sq, sk = int(rng.integers(1, 150)), int(rng.integers(1, 200))
        causal = bool(rng.integers(0, 2))
        sigma = float(rng.choice([0.5, 1.0, 2.0]))
        q = (rng.standard_normal(bh * sq * d) * sigma).astype(np.float32)
        k = (rng.standard_normal(bh * sk * d) * sigma).astype(np.float32)
        v = rng.uniform(-1, 1, bh * sk * d).astype(np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        got = {}
        for variant in ALL_VARIANTS:
            plan = fa.describe_launch(variant, 1, bh, sq, sk, d, causal)
            tag = f"fuzz {case}: v{variant} ({bh},{sq},{sk},{d},{causal}) sigma={sigma} {plan}"
            print("[case]", tag, flush=True)
            assert ("_dreg_" if d <= 4096 else "_dany_") in plan, plan
            got[variant] = _device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=64)
            assert_parity(got[variant], want, tag)
        assert np.array_equal(got[2], got[3]), case


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_multihead_matches_per_head(variant):
    batch, heads, seq_q, seq_k, d = 2, 3, 37, 50, 16
    q = random_vec(batch * heads * seq_q * d, 21)
    k = random_vec(batch * heads * seq_k * d, 22)
    v = random_vec(batch * heads * seq_k * d, 23)
    out = np.zeros(batch * heads * seq_q * d, dtype=np.float32)
    fa.MULTIHEAD_VARIANTS[variant](q, k, v, batch, heads, seq_q, seq_k, d,
                                   fa.FlashAttentionConfig(8, 12, True), out)
    assert_parity(out, cpu_v2(q, k, v, batch * heads, seq_q, seq_k, d, True), f"multihead v{variant}")
    for bh in range(batch * heads):
        sl_q = slice(bh * seq_q * d, (bh + 1) * seq_q * d)
        sl_k = slice(bh * seq_k * d, (bh + 1) * seq_k * d)
        want = oracle.naive_f64(q[sl_q], k[sl_k], v[sl_k], seq_q, seq_k, d, True)
        assert max_abs_diff(out[sl_q], want) < NAIVE_TOL


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_causal_first_query_equals_first_value_row(variant):
    # tests/correctness.rs:240-263: row 0 attends only to key 0.
    seq, d = 256, 64
    q, k, v = random_vec(seq * d, 30), random_vec(seq * d, 31), random_vec(seq * d, 32)
    for br, bc in [(64, 128), (32, 32), (1024, 1024), (1, 1)]:
        out = np.zeros(seq * d, dtype=np.float32)
        fa.VARIANTS[variant](q, k, v, seq, seq, d, fa.FlashAttentionConfig(br, bc, True), out)
        assert max_abs_diff(out[:d], v[:d]) < 1e-6


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_single_key_returns_first_value_row(variant):
    # seq_k == 1: softmax over one key is 1 for every row.
    seq_q, d = 300, 128
    q, k, v = normal_vec(seq_q * d, 5), normal_vec(d, 6), normal_vec(d, 7)
    out = np.zeros(seq_q * d, dtype=np.float32)
    fa.VARIANTS[variant](q, k, v, seq_q, 1, d, fa.FlashAttentionConfig(), out)
    assert max_abs_diff(out.reshape(seq_q, d), np.broadcast_to(v, (seq_q, d))) < 1e-6


def test_output_is_finite_and_deterministic():
    seq, d = 40, 32
    q, k, v = random_vec(seq * d, 10), random_vec(seq * d, 11), random_vec(seq * d, 12)
    for variant in ALL_VARIANTS:
        a = np.zeros(seq * d, dtype=np.float32)
        b = np.zeros(seq * d, dtype=np.float32)
        cfg = fa.FlashAttentionConfig(causal=True)
        fa.VARIANTS[variant](q, k, v, seq, seq, d, cfg, a)
        fa.VARIANTS[variant](q, k, v, seq, seq, d, cfg, b)
        assert np.all(np.isfinite(a))
        assert np.array_equal(a, b), f"v{variant} not deterministic"


def test_v1_v2_v3_mutually_agree():
    # tests/correctness.rs:299-375 (v2 and v3 must agree to 1e-5 there).
    for seq_q, seq_k, d, br, bc, causal in [(64, 64, 64, 32, 32, False), (97, 131, 17, 32, 40, True),
                                            (5, 5, 8, 64, 64, True), (200, 200, 128, 64, 128, True),
                                            (700, 650, 128, 64, 128, True)]:
        q, k, v = random_vec(seq_q * d, 1), random_vec(seq_k * d, 2), random_vec(seq_k * d, 3)
        outs = {}
        for variant in ALL_VARIANTS:
            outs[variant] = np.zeros(seq_q * d, dtype=np.float32)
            fa.VARIANTS[variant](q, k, v, seq_q, seq_k, d, fa.FlashAttentionConfig(br, bc, causal),
                                 outs[variant])
        assert_parity(outs[1], outs[2], "v1 vs v2")
        assert_parity(outs[3], outs[2], "v3 vs v2")
        assert max_abs_diff(outs[2], outs[3]) < 1e-5


def test_shape_mismatches_raise():
    seq_q, seq_k, d = 4, 4, 8
    q, k, v = random_vec(seq_q * d, 1), random_vec(seq_k * d, 2), random_vec(seq_k * d, 3)
    cfg = fa.FlashAttentionConfig()
    for variant in ALL_VARIANTS:
        f = fa.VARIANTS[variant]
        for args, msg in [((q[:-1], k, v), "q shape mismatch"), ((q, k[:-1], v), "k shape mismatch"),
                          ((q, k, v[:-1]), "v shape mismatch")]:
            with pytest.raises(fa.ShapeMismatch, match=msg):
                f(*args, seq_q, seq_k, d, cfg, np.zeros(seq_q * d, dtype=np.float32))
        with pytest.raises(fa.ShapeMismatch, match="out shape mismatch"):
            f(q, k, v, seq_q, seq_k, d, cfg, np.zeros(seq_q * d - 1, dtype=np.float32))


def test_zero_sized_dimensions_leave_out_untouched():
    d = 8
    for variant in ALL_VARIANTS:
        f = fa.VARIANTS[variant]
        out = np.full(4 * d, 12.5, dtype=np.float32)
        f(random_vec(4 * d, 4), np.zeros(0, np.float32), np.zeros(0, np.float32), 4, 0, d,
          fa.FlashAttentionConfig(), out)
        assert np.all(out == 12.5)
        f(np.zeros(0, np.float32), random_vec(4 * d, 2), random_vec(4 * d, 3), 0, 4, d,
          fa.FlashAttentionConfig(), np.zeros(0, np.float32))


def test_differential_fuzz_small_shapes():
    # fuzz/fuzz_targets/flash_attention.rs:89-126: random small shapes and
    # magnitudes 10^0..10^6, v1/v2/v3 and the oracle must agree.
    rng = np.random.default_rng(1234)
    for it in range(60):
        seq_q, seq_k, d = (int(x) for x in rng.integers(1, 21, 3))
        d = int(rng.integers(1, 17))
        causal = bool(rng.integers(0, 2))
        mag = float(10.0 ** rng.integers(0, 7))
        q = (rng.uniform(-1, 1, seq_q * d) * mag).astype(np.float32)
        k = (rng.uniform(-1, 1, seq_k * d) * mag).astype(np.float32)
        v = (rng.uniform(-1, 1, seq_k * d) * mag).astype(np.float32)
        want = cpu_v2(q, k, v, 1, seq_q, seq_k, d, causal)
        for variant in ALL_VARIANTS:
            out = np.zeros(seq_q * d, dtype=np.float32)
            fa.VARIANTS[variant](q, k, v, seq_q, seq_k, d, fa.FlashAttentionConfig(causal=causal), out)
            assert np.array_equal(np.isfinite(out), np.isfinite(want)), f"it={it}"
            tol = 1e-1 * (np.maximum(np.abs(out), np.abs(want)) + 1.0)
            assert np.all(np.abs(out - want) < tol), f"it={it} v{variant} shape=({seq_q},{seq_k},{d}) mag={mag}"


def test_differential_fuzz_split_paths():
    """The fuzzer's magnitudes (10^0..10^6) and its tolerance on the shapes
    that take the split paths: the row-streaming decode (seq_q <= 4), the
    16-row split-KV tiles (decode shapes and small prefills) and the key-split
    prefill, through AUTO and forced paths."""
    rng = np.random.default_rng(4321)
    for it in range(24):
        sq = int(rng.choice([1, 2, 3, 4, 9, 16, 40, 300]))
        sk = int(rng.integers(256, 3000))
        d = int(rng.choice([8, 20, 32, 64, 100, 128, 256]))
        bh = int(rng.integers(1, 4))
        causal = bool(rng.integers(0, 2))
        mag = float(10.0 ** rng.integers(0, 7))
        q = (rng.uniform(-1, 1, bh * sq * d) * mag).astype(np.float32)
        k = (rng.uniform(-1, 1, bh * sk * d) * mag).astype(np.float32)
        v = (rng.uniform(-1, 1, bh * sk * d) * mag).astype(np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        paths = [(fa.PATH_AUTO, 0), (fa.PATH_SPLITKV, 0), (fa.PATH_PREFILL, 3)]
        if sq <= 4 and d % 4 == 0:
            paths.append((fa.PATH_SPLITKV_ROWS, 0))
        for path, splits in paths:
            outs = {}
            for variant in (1, 3):   # v1's split kernels (per-block normalisation) and v3's
                tag = f"it={it} v{variant} path={path} ({bh},{sq},{sk},{d},{causal}) mag={mag}"
                print("[case]", tag, flush=True)
                out = outs[variant] = _device_run(variant, q, k, v, bh, sq, sk, d, causal, path, splits, guard=64)
                assert np.array_equal(np.isfinite(out), np.isfinite(want)), tag
                tol = 1e-1 * (np.maximum(np.abs(out), np.abs(want)) + 1.0)
                assert np.all(np.abs(out - want) < tol), tag
            if mag == 1.0:
                assert_parity(outs[1], outs[3], f"it={it} v1 vs v3 path={path}")


def test_differential_fuzz_new_paths():
    """Random shapes through the column-group kernels (d_head 257..2048), the
    stream split (forced, random workgroup counts) and the LDS-staged split-KV
    tiles (d_head 64 / 128), v2 and v3 against the oracle's CPU v2, with the
    fuzzer's magnitudes for the split paths (fuzz/fuzz_targets/flash_attention.rs:89-126)
    and the parity bar for unit-scale inputs."""
    rng = np.random.default_rng(5150)
    for it in range(30):
        kind = it % 3
        bh = int(rng.integers(1, 4))
        causal = bool(rng.integers(0, 2))
        if kind == 0:      # wide heads
            d = int(rng.integers(257, 2049))
            sq, sk = int(rng.integers(1, 300)), int(rng.integers(1, 400))
            path, splits, mag = fa.PATH_AUTO, 0, 1.0
        elif kind == 1:    # stream split
            d = int(rng.choice([8, 33, 64, 100, 128, 200, 256, 300, 512]))
            sq, sk = int(rng.integers(1, 700)), int(rng.integers(1, 900))
            path, splits, mag = fa.PATH_STREAM, int(rng.integers(0, 300)), float(10.0 ** rng.integers(0, 4))
        else:              # LDS-staged decode tiles
            d = int(rng.choice([64, 128, 68, 96, 124]))
            sq, sk = int(rng.integers(5, 64)), int(rng.integers(300, 5000))
            path, splits, mag = fa.PATH_SPLITKV, int(rng.integers(0, 40)), float(10.0 ** rng.integers(0, 4))
        q = (rng.uniform(-1, 1, bh * sq * d) * mag).astype(np.float32)
        k = (rng.uniform(-1, 1, bh * sk * d) * mag).astype(np.float32)
        v = (rng.uniform(-1, 1, bh * sk * d)).astype(np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for variant in ALL_VARIANTS:
            plan = fa.describe_launch(variant, 1, bh, sq, sk, d, causal, path, splits)
            tag = f"it={it} v{variant} ({bh},{sq},{sk},{d},{causal}) mag={mag}: {plan}"
            print("[case]", tag, flush=True)
            out = _device_run(variant, q, k, v, bh, sq, sk, d, causal, path, splits, guard=64)
            if mag == 1.0:
                assert_parity(out, want, tag)
            else:
                assert np.array_equal(np.isfinite(out), np.isfinite(want)), tag
                tol = 1e-1 * (np.maximum(np.abs(out), np.abs(want)) + 1.0)
                assert np.all(np.abs(out - want) < tol), tag


# ---------------------------------------------------------------------------
# BASELINE.json configs
# ---------------------------------------------------------------------------

def _qkv(bh, sq, sk, d, qk_sigma=1.0, v_uniform=False):
    q = normal_vec(bh * sq * d, 1, qk_sigma)
    k = normal_vec(bh * sk * d, 2, qk_sigma)
    v = uniform_vec(bh * sk * d, 3) if v_uniform else normal_vec(bh * sk * d, 3)
    return q, k, v


def test_config1_single_head_256():
    sq = sk = 256
    d = 64
    q, k, v = _qkv(1, sq, sk, d)
    want = cpu_v2(q, k, v, 1, sq, sk, d, False)
    out = np.zeros(sq * d, dtype=np.float32)
    fa.flash_attention(q, k, v, sq, sk, d, fa.FlashAttentionConfig(), out)
    assert_parity(out, want, "config 1")
    assert max_abs_diff(out, attention_f64(q, k, v, sq, sk, d, False)) < 2e-5
    for variant in ALL_VARIANTS:
        out = np.zeros(sq * d, dtype=np.float32)
        fa.VARIANTS[variant](q, k, v, sq, sk, d, fa.FlashAttentionConfig(), out)
        assert_parity(out, want, f"config 1 v{variant}")


@pytest.mark.parametrize("variant", ALL_VARIANTS)
def test_config2_prefill_32h_2048_d128_causal(variant):
    bh, s, d = 32, 2048, 128
    q, k, v = _qkv(bh, s, s, d)
    out = np.zeros(bh * s * d, dtype=np.float32)
    fa.MULTIHEAD_VARIANTS[variant](q, k, v, 1, bh, s, s, d, fa.FlashAttentionConfig(causal=True), out)
    assert_parity(out, cpu_v2(q, k, v, bh, s, s, d, True), f"config 2 v{variant}")


def test_config4_decode_split_kv():
    bh, sk, d = 32, 32768, 128
    k = normal_vec(bh * sk * d, 2)
    v = normal_vec(bh * sk * d, 3)
    for sq in (1, 16):
        q = normal_vec(bh * sq * d, 1)
        assert "fa_decode" in fa.describe_launch(2, 1, bh, sq, sk, d, False)
        want = cpu_v2(q, k, v, bh, sq, sk, d, False)
        for variant in ALL_VARIANTS:
            out = np.zeros(bh * sq * d, dtype=np.float32)
            fa.MULTIHEAD_VARIANTS[variant](q, k, v, 1, bh, sq, sk, d, fa.FlashAttentionConfig(), out)
            assert_parity(out, want, f"config 4 seq_q={sq} v{variant}")


def test_config5_cross_attention_peaky_d256():
    bh, sq, sk, d = 16, 4096, 1024, 256
    q, k, v = _qkv(bh, sq, sk, d, qk_sigma=3.0, v_uniform=True)
    want = cpu_v2(q, k, v, bh, sq, sk, d, False)
    for variant in ALL_VARIANTS:
        out = np.zeros(bh * sq * d, dtype=np.float32)
        fa.MULTIHEAD_VARIANTS[variant](q, k, v, 1, bh, sq, sk, d, fa.FlashAttentionConfig(), out)
        assert_parity(out, want, f"config 5 v{variant}")


def test_config5c_causal_1000_remainders_d256():
    bh, s, d = 16, 1000, 256
    q, k, v = _qkv(bh, s, s, d, qk_sigma=3.0, v_uniform=True)
    want = cpu_v2(q, k, v, bh, s, s, d, True)
    for variant in ALL_VARIANTS:
        out = np.zeros(bh * s * d, dtype=np.float32)
        fa.MULTIHEAD_VARIANTS[variant](q, k, v, 1, bh, s, s, d, fa.FlashAttentionConfig(causal=True), out)
        assert_parity(out, want, f"config 5c v{variant}")


# ---------------------------------------------------------------------------
# Golden vectors, split-KV, device API
# ---------------------------------------------------------------------------

def test_golden_vectors():
    from golden.make_golden import load as load_golden
    for name, (bh, sq, sk, d, causal, q, k, v, exp) in load_golden().items():
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for variant in ALL_VARIANTS:
            out = np.zeros(bh * sq * d, dtype=np.float32)
            fa.MULTIHEAD_VARIANTS[variant](q, k, v, 1, bh, sq, sk, d, fa.FlashAttentionConfig(causal=causal), out)
            tol = 2e-5 if name.startswith("peaky") else 2e-6
            assert max_abs_diff(out, exp) < tol, (name, variant)
            assert_parity(out, want, f"golden {name} v{variant}")


def _torch():
    import torch
    return torch


def _device_run(variant, q, k, v, bh, sq, sk, d, causal, path=fa.PATH_AUTO, splits=0, scale=None, guard=0):
    """Run on device tensors; `guard` floats of sentinel around the output."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    tq = torch.from_numpy(q).to(dev)
    tk = torch.from_numpy(k).to(dev)
    tv = torch.from_numpy(v).to(dev)
    buf = torch.full((bh * sq * d + 2 * guard,), 12.5, device=dev)
    out = buf[guard:guard + bh * sq * d]
    fa.attention_device(variant, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, bh, sq, sk, d, causal,
                        out.data_ptr(), torch.cuda.current_stream().cuda_stream, softmax_scale=scale, path=path,
                        num_splits=splits)
    torch.cuda.synchronize()
    host = buf.cpu().numpy()
    if guard:
        assert np.all(host[:guard] == 12.5) and np.all(host[-guard:] == 12.5), "write outside out"
    return host[guard:guard + bh * sq * d]


def test_split_kv_matches_oracle_and_prefill():
    rng = np.random.default_rng(77)
    cases = [(1, 1, 700, 128, False), (3, 16, 1000, 128, False), (2, 5, 333, 64, True), (1, 40, 513, 32, True),
             (2, 64, 2048, 256, False), (1, 17, 129, 17, False), (4, 1, 4096, 40, False), (1, 33, 96, 128, True)]
    for bh, sq, sk, d, causal in cases:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        pre = _device_run(2, q, k, v, bh, sq, sk, d, causal, fa.PATH_PREFILL, guard=64)
        assert_parity(pre, want, f"prefill {bh},{sq},{sk},{d},{causal}")
        for splits in (0, 1, 2, 3, 7):
            for variant in ALL_VARIANTS:
                got = _device_run(variant, q, k, v, bh, sq, sk, d, causal, fa.PATH_SPLITKV, splits, guard=64)
                assert_parity(got, want, f"split-kv v{variant} splits={splits} {bh},{sq},{sk},{d},{causal}")


def test_row_streaming_decode_matches_oracle():
    """Row-streaming split-KV (seq_q <= 4, K/V read as whole rows, dot
    products reduce-scattered across lanes): every padded head size, d below
    the padded size (lanes past d), key ranges that end inside a key block and
    splits whose waves get no keys, causal (only keys <= query row visible),
    peaky logits, and a reference that moves mid-sequence."""
    rng = np.random.default_rng(79)
    cases = [(1, 1, 700, 128, False, 1.0), (3, 2, 1000, 128, False, 1.0), (2, 3, 333, 64, True, 1.0),
             (1, 4, 513, 32, False, 1.0), (2, 1, 2048, 256, False, 1.0), (1, 3, 129, 40, False, 1.0),
             (4, 1, 4096, 100, False, 3.0), (2, 4, 96, 128, True, 1.0), (2, 2, 1000, 256, False, 3.0),
             (1, 1, 5, 64, False, 1.0), (3, 4, 777, 20, True, 1.0)]
    for bh, sq, sk, d, causal, sigma in cases:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32) * np.float32(sigma)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32) * np.float32(sigma)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for splits in (0, 1, 2, 3, 7, 40):
            for variant in ALL_VARIANTS:
                tag = f"rows v{variant} splits={splits} {bh},{sq},{sk},{d},{causal},sigma={sigma}"
                print("[case]", tag, flush=True)
                got = _device_run(variant, q, k, v, bh, sq, sk, d, causal, fa.PATH_SPLITKV_ROWS, splits, guard=64)
                assert_parity(got, want, tag)
        desc = fa.describe_launch(2, 1, bh, sq, sk, d, causal, fa.PATH_SPLITKV_ROWS)
        assert desc.startswith("fa_decode_rows_"), desc
    # the key scale steps up after 64 keys: the lazy reference moves mid-sequence
    bh, sk, d = 4, 3000, 128
    for sq in (1, 4):
        q = rng.standard_normal((bh, sq, d), dtype=np.float32)
        ramp = np.where(np.arange(sk) < 64, 0.05, 2.4).astype(np.float32)[None, :, None]
        k = (rng.standard_normal((bh, sk, d), dtype=np.float32) * ramp).astype(np.float32).ravel()
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        q = q.ravel()
        want = cpu_v2(q, k, v, bh, sq, sk, d, False)
        for splits in (0, 1, 5):
            got = _device_run(2, q, k, v, bh, sq, sk, d, False, fa.PATH_SPLITKV_ROWS, splits, guard=64)
            assert_parity(got, want, f"rows rising sq={sq} splits={splits}")
    # AUTO picks it for decode shapes; shapes it cannot take are refused
    assert fa.describe_launch(2, 1, 32, 1, 32768, 128, False).startswith("fa_decode_rows_d128_q1")
    assert fa.describe_launch(3, 1, 32, 3, 32768, 64, False).startswith("fa_decode_rows_d64_q4")
    assert fa.describe_launch(2, 1, 32, 16, 32768, 128, False).startswith("fa_decode_d128")
    with pytest.raises(fa.FaError):
        fa.describe_launch(2, 1, 4, 5, 1000, 128, False, fa.PATH_SPLITKV_ROWS)   # seq_q > 4
    with pytest.raises(fa.FaError):
        fa.describe_launch(2, 1, 4, 1, 1000, 17, False, fa.PATH_SPLITKV_ROWS)    # d % 4 != 0


def test_single_split_decode_writes_rows_directly():
    """One key split: the decode kernels write the normalised rows themselves -- no workspace,
    no merge launch -- for the 16-row tiles (every padded width, causal and
    ragged) and the row-streaming kernel (1-4 rows)."""
    rng = np.random.default_rng(31)
    cases = [(fa.PATH_SPLITKV, 2, 16, 700, 64, False), (fa.PATH_SPLITKV, 1, 5, 333, 17, True),
             (fa.PATH_SPLITKV, 3, 40, 300, 128, True), (fa.PATH_SPLITKV, 1, 20, 257, 256, False),
             (fa.PATH_SPLITKV, 2, 9, 129, 33, False), (fa.PATH_SPLITKV_ROWS, 4, 1, 900, 128, False),
             (fa.PATH_SPLITKV_ROWS, 2, 3, 70, 64, True), (fa.PATH_SPLITKV_ROWS, 1, 4, 513, 256, False),
             (fa.PATH_SPLITKV_ROWS, 3, 2, 64, 32, True)]
    for path, bh, sq, sk, d, causal in cases:
        plan = fa.describe_launch(2, 1, bh, sq, sk, d, causal, path, 1)
        assert "fa_decode" in plan and "fa_merge" not in plan and "workspace" not in plan, plan
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for variant in ALL_VARIANTS:
            tag = f"v{variant} {plan} ({bh},{sq},{sk},{d},{causal})"
            print("[case]", tag, flush=True)
            assert_parity(_device_run(variant, q, k, v, bh, sq, sk, d, causal, path, 1, guard=64), want, tag)


def test_batched_decode_steps_take_split_kv():
    """Decode steps of many slices (a grid of at least one prefill block per
    CU) run the decode kernels, in one split when the slices alone fill the
    GPU: the row kernel (1-4 queries) and the 16-row tiles (up to 32), v2 and
    v3 against the oracle, with a guard around the output."""
    rng = np.random.default_rng(47)
    for bh, sq, sk, d, causal, kernel in [(512, 1, 1024, 128, False, "fa_decode_rows_d128_q1 grid=512x1x1"),
                                          (300, 3, 700, 64, True, "fa_decode_rows_d64_q4 grid=300x1x1"),
                                          (256, 32, 600, 128, False, "fa_decode_d128_2 grid=512x1x1"),
                                          (260, 20, 530, 40, True, "fa_decode_d64_2 grid=520x1x1"),
                                          # more slices than a 3-D grid's y / z dimension holds
                                          (70000, 1, 64, 32, False, "fa_decode_rows_d32_q1 grid=70000x1x1")]:
        plan = fa.describe_launch(2, 1, bh, sq, sk, d, causal)
        assert plan.startswith(kernel) and "fa_merge" not in plan, plan
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for variant in ALL_VARIANTS:
            tag = f"v{variant} {plan}"
            print("[case]", tag, flush=True)
            assert_parity(_device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=64), want, tag)


def test_small_prefill_on_split_kv_tiles_matches_oracle():
    """Grids smaller than the GPU with at most 128 16-row tiles x heads and
    256+ keys run on the split-KV 16-row tiles (AUTO): long query ranges,
    causal and ragged shapes, every padded head size; v2 and v3 agree."""
    rng = np.random.default_rng(81)
    cases = [(1, 2048, 2048, 128, True), (1, 1000, 1000, 128, False), (2, 300, 700, 64, True),
             (4, 256, 1000, 256, True), (1, 777, 300, 40, False), (3, 500, 256, 32, True)]
    for bh, sq, sk, d, causal in cases:
        plan = fa.describe_launch(2, 1, bh, sq, sk, d, causal)
        assert plan.startswith("fa_decode_d"), plan
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for variant in ALL_VARIANTS:
            tag = f"small prefill v{variant} {bh},{sq},{sk},{d},{causal}"
            print("[case]", tag, plan, flush=True)
            assert_parity(_device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=64), want, tag)


def test_key_split_prefill_matches_oracle():
    """v1/v2/v3 query-block kernels with each block's keys divided over several
    workgroups and the partials merged (forced here; chosen automatically on
    grids smaller than the GPU)."""
    rng = np.random.default_rng(78)
    cases = [(1, 1000, 1000, 256, True), (2, 300, 700, 64, False), (1, 700, 300, 128, True),
             (3, 129, 1025, 32, True), (1, 257, 513, 17, False), (2, 200, 2000, 128, False)]
    for bh, sq, sk, d, causal in cases:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for splits in (2, 3, 5, 16):
            for variant in ALL_VARIANTS:
                tag = f"key-split v{variant} splits={splits} {bh},{sq},{sk},{d},{causal}"
                print("[case]", tag, flush=True)
                got = _device_run(variant, q, k, v, bh, sq, sk, d, causal, fa.PATH_PREFILL, splits, guard=64)
                assert_parity(got, want, tag)
        # automatic choice (small grid) and its determinism
        for variant in ALL_VARIANTS:
            a = _device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=64)
            b = _device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=64)
            assert np.array_equal(a, b)
            assert_parity(a, want, f"auto v{variant} {bh},{sq},{sk},{d},{causal}")


def test_stream_split_prefill_matches_oracle():
    """v1/v2/v3 query-block kernels with the stream split: the key stages of all
    (slice, query block) pairs cut into equal runs, one per workgroup, runs
    crossing block and slice boundaries, shared blocks merged (forced here
    with several workgroup counts; chosen automatically for small causal
    grids such as config 5c).  Ragged ends, non-causal, seq_q > seq_k, every
    kernel width."""
    rng = np.random.default_rng(79)
    cases = [(16, 1000, 1000, 256, True), (3, 300, 700, 64, False), (2, 700, 300, 128, True),
             (3, 129, 1025, 32, True), (1, 257, 513, 17, False), (2, 600, 600, 512, True), (1, 100, 900, 1024, True),
             (5, 77, 77, 128, True)]
    for bh, sq, sk, d, causal in cases:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for splits in (0, 1, 3, 7, 64):
            for variant in ALL_VARIANTS:
                plan = fa.describe_launch(variant, 1, bh, sq, sk, d, causal, fa.PATH_STREAM, splits)
                tag = f"stream v{variant} workgroups={splits} {bh},{sq},{sk},{d},{causal}: {plan}"
                print("[case]", tag, flush=True)
                assert "stream_per=" in plan, tag
                got = _device_run(variant, q, k, v, bh, sq, sk, d, causal, fa.PATH_STREAM, splits, guard=64)
                assert_parity(got, want, tag)
    # v1 splits with every block visiting all keys (no causal skip)
    assert "stream_per=16" in fa.describe_launch(1, 1, 16, 1000, 1000, 256, True, fa.PATH_STREAM)
    assert "stream_per=18" in fa.describe_launch(3, 1, 16, 1000, 1000, 256, True)   # config 5c: automatic


def test_misaligned_device_pointers_match_oracle():
    """Device pointers 4 bytes past a 16-byte boundary (Q, K, V and out each
    offset by one float, d % 4 == 0): the planner takes the scalar loaders and
    the merges' element-wise stores; every path (automatic, prefill, key split,
    stream split, split-KV tiles) and variant against the oracle, with
    sentinels around out."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(83)
    cases = [(1, 1000, 1000, 256, True), (3, 300, 700, 64, False), (2, 200, 200, 128, True),
             (4, 1, 2048, 128, False), (2, 16, 1500, 64, False), (1, 256, 256, 64, False)]
    for bh, sq, sk, d, causal in cases:
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        tq, tk, tv = (torch.from_numpy(np.concatenate([np.zeros(1, np.float32), x])).to(dev) for x in (q, k, v))
        for path, splits in ((fa.PATH_AUTO, 0), (fa.PATH_PREFILL, 0), (fa.PATH_PREFILL, 3), (fa.PATH_STREAM, 0),
                             (fa.PATH_SPLITKV, 2)):
            for variant in ALL_VARIANTS:
                # (describe_launch plans for aligned pointers; these calls take the scalar loaders)
                tag = (f"misaligned v{variant} path={path} splits={splits} {bh},{sq},{sk},{d},{causal}; aligned plan: "
                       f"{fa.describe_launch(variant, 1, bh, sq, sk, d, causal, path, splits)}")
                print("[case]", tag, flush=True)
                buf = torch.full((bh * sq * d + 2 + 64,), 12.5, device=dev)
                out = buf[1:1 + bh * sq * d]
                fa.attention_device(variant, tq[1:].data_ptr(), tk[1:].data_ptr(), tv[1:].data_ptr(), 1, bh, sq, sk,
                                    d, causal, out.data_ptr(), torch.cuda.current_stream().cuda_stream, path=path,
                                    num_splits=splits)
                torch.cuda.synchronize()
                host = buf.cpu().numpy()
                assert host[0] == 12.5 and np.all(host[1 + bh * sq * d:] == 12.5), "write outside out: " + tag
                assert_parity(host[1:1 + bh * sq * d], want, tag)


def test_two_block_workgroups_match_oracle():
    """f32 v3 grids whose block pairs fill whole rounds of the GPU run query
    blocks nqb-1-r and r in one workgroup, the second block's loads issued
    during the first's last step.  Ragged last blocks, non-causal, and key
    ranges that end inside a stage; v2 (one block per workgroup) agrees."""
    rng = np.random.default_rng(91)
    num_cus = 256   # MI355X; the pairing needs (nqb / 2) * bh to be a multiple of it
    for sq, sk, d, causal in [(200, 300, 128, True), (256, 256, 128, False), (250, 190, 128, False),
                              (130, 1000, 128, True)]:
        bh = num_cus   # nqb = 2: one pair per (batch, head)
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        tag = f"two-block {bh},{sq},{sk},{d},{causal}"
        print("[case]", tag, flush=True)
        assert "two_blocks" in fa.describe_launch(3, 1, bh, sq, sk, d, causal), tag
        assert "two_blocks" not in fa.describe_launch(2, 1, bh, sq, sk, d, causal)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        got = _device_run(3, q, k, v, bh, sq, sk, d, causal, guard=64)
        assert_parity(got, want, tag)
        assert max_abs_diff(got, _device_run(2, q, k, v, bh, sq, sk, d, causal, guard=64)) < 2e-5, tag
    # padded d_head (d < D) and d_head < 128 keep one block per workgroup
    assert "two_blocks" not in fa.describe_launch(3, 1, 256, 200, 300, 100, True)
    assert "two_blocks" not in fa.describe_launch(3, 1, 256, 200, 300, 64, True)


def test_v3_first_stage_edges_match_oracle():
    """v3's DMA kernels at D = 128 and 256 load Q after the first stages'
    DMA (buffer loads; rows past seq_q and columns past d read as zeros) and
    always issue K(0), V(0) and K(1), repeating stage 0 when there is no
    second stage.  Key ranges of one stage and of one key, ragged query
    tiles, padded columns, unsplit and key-split segments (which start
    mid-range), against the oracle's CPU v2."""
    rng = np.random.default_rng(93)
    for d in (100, 128, 200, 256):
        D = 128 if d <= 128 else 256
        for sq, sk in ((70, 1), (70, 5), (70, 64), (130, 65), (16, 64), (150, 200)):
            bh = 2
            q = rng.standard_normal(bh * sq * d, dtype=np.float32)
            k = rng.standard_normal(bh * sk * d, dtype=np.float32)
            v = rng.standard_normal(bh * sk * d, dtype=np.float32)
            for causal in (False, True):
                want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
                for splits in (1, 2):
                    plan = fa.describe_launch(3, 1, bh, sq, sk, d, causal, fa.PATH_PREFILL, splits)
                    tag = f"v3 first stage {bh},{sq},{sk},{d},{causal} splits={splits}: {plan}"
                    print("[case]", tag, flush=True)
                    assert plan.startswith(f"fa_prefill_v3_d{D}_2"), tag
                    got = _device_run(3, q, k, v, bh, sq, sk, d, causal, fa.PATH_PREFILL, splits, guard=64)
                    assert_parity(got, want, tag)


def test_reference_moves_mid_sequence():
    """Keys 0..63 with tiny logits (std 0.05) and later keys with large ones
    (std 2.4): a row's maximum jumps past the lazy 2^8 threshold after the
    first 64-key stage (checked on the CPU for 30-98 % of the rows), so the
    reference moves mid-sequence and the O / l rescale and the -m starting
    accumulator run there, including on the two-block grid (first rows of
    this list)."""
    rng = np.random.default_rng(5)
    for bh, sq, sk, d, causal, variant in [(256, 256, 256, 128, True, 3), (256, 256, 256, 128, False, 3),
                                           (4, 300, 700, 128, True, 2), (4, 300, 700, 64, False, 3),
                                           (2, 200, 640, 256, False, 3)]:
        q = rng.standard_normal((bh, sq, d), dtype=np.float32)
        ramp = np.where(np.arange(sk) < 64, 0.05, 2.4).astype(np.float32)[None, :, None]
        k = (rng.standard_normal((bh, sk, d), dtype=np.float32) * ramp).astype(np.float32)
        v = rng.standard_normal((bh, sk, d), dtype=np.float32)
        q, k, v = q.ravel(), k.ravel(), v.ravel()
        tag = f"rising v{variant} {bh},{sq},{sk},{d},{causal}"
        print("[case]", tag, flush=True)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        got = _device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=64)
        assert_parity(got, want, tag)


def test_device_api_bounds_and_determinism():
    for bh, sq, sk, d, causal in [(3, 130, 77, 128, True), (2, 257, 300, 64, False), (1, 129, 129, 256, True),
                                  (2, 100, 50, 20, False), (5, 3, 1000, 128, False)]:
        q, k, v = random_vec(bh * sq * d, 1), random_vec(bh * sk * d, 2), random_vec(bh * sk * d, 3)
        want = cpu_v2(q, k, v, bh, sq, sk, d, causal)
        for variant in ALL_VARIANTS:
            a = _device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=256)
            b = _device_run(variant, q, k, v, bh, sq, sk, d, causal, guard=256)
            assert np.array_equal(a, b), f"v{variant} not deterministic"
            assert_parity(a, want, f"device v{variant} {bh},{sq},{sk},{d},{causal}")


def test_explicit_softmax_scale_extension():
    bh, sq, sk, d = 2, 90, 140, 64
    q, k, v = random_vec(bh * sq * d, 1), random_vec(bh * sk * d, 2), random_vec(bh * sk * d, 3)
    scale = 0.3
    # attention with scale s equals default attention on Q * (s * sqrt(d))
    q2 = (q.astype(np.float64) * scale * np.sqrt(d)).astype(np.float32)
    want = np.concatenate([attention_f64(q2[h * sq * d:(h + 1) * sq * d], k[h * sk * d:(h + 1) * sk * d],
                                         v[h * sk * d:(h + 1) * sk * d], sq, sk, d, True) for h in range(bh)])
    for variant in ALL_VARIANTS:
        got = _device_run(variant, q, k, v, bh, sq, sk, d, True, scale=scale)
        assert max_abs_diff(got, want) < 1e-5


def test_explicit_softmax_scale_on_every_split_path():
    """The explicit scale reaches every kernel and merge: prefill, key split,
    stream split (register-order tiles merged by fa_merge_tiles at D = 64, 128,
    256; rows by fa_merge at D = 32) and split-KV tiles, every variant, against
    float64 attention on Q * (s * sqrt(d)) (the same attention)."""
    rng = np.random.default_rng(89)
    for bh, sq, sk, d, causal, scale in ((2, 300, 500, 64, True, 0.3), (1, 200, 700, 128, False, 0.05),
                                         (1, 260, 260, 256, True, 0.02), (2, 100, 400, 32, True, 0.5)):
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        q2 = (q.astype(np.float64) * scale * np.sqrt(d)).astype(np.float32)
        want = np.concatenate([attention_f64(q2[h * sq * d:(h + 1) * sq * d], k[h * sk * d:(h + 1) * sk * d],
                                             v[h * sk * d:(h + 1) * sk * d], sq, sk, d, causal) for h in range(bh)])
        for path, splits in ((fa.PATH_PREFILL, 0), (fa.PATH_PREFILL, 3), (fa.PATH_STREAM, 0), (fa.PATH_SPLITKV, 2)):
            for variant in ALL_VARIANTS:
                tag = (f"scale {scale} v{variant} path={path} splits={splits} {bh},{sq},{sk},{d},{causal}: "
                       f"{fa.describe_launch(variant, 1, bh, sq, sk, d, causal, path, splits)}")
                print("[case]", tag, flush=True)
                got = _device_run(variant, q, k, v, bh, sq, sk, d, causal, path, splits, scale=scale, guard=64)
                err = max_abs_diff(got, want)
                assert err < 2e-5, f"{tag}: max-abs {err:.3g}"


def test_long_context_config3_properties():
    # 8 heads x 16384^2 causal: full parity against the CPU v2 on a sample of
    # rows (float64 naive per row) plus the causal row-0 known answer.
    bh, s, d = 8, 16384, 128
    q, k, v = _qkv(bh, s, s, d)
    rows = [0, 1, 127, 128, 4095, 8191, 12345, 16383]
    for variant in (1, 2, 3):
        out = np.zeros(bh * s * d, dtype=np.float32)
        fa.MULTIHEAD_VARIANTS[variant](q, k, v, 1, bh, s, s, d, fa.FlashAttentionConfig(causal=True), out)
        assert np.all(np.isfinite(out))
        for h in (0, 7):
            sl_q = slice(h * s * d, (h + 1) * s * d)
            o = out[sl_q].reshape(s, d)
            assert max_abs_diff(o[0], v[h * s * d:h * s * d + d]) < 1e-6
            for r in rows:
                ref = oracle.naive_f64(q[sl_q], k[sl_q], v[sl_q], s, s, d, True, r, 1)
                assert max_abs_diff(o[r], ref) < 2e-5, (variant, h, r)


def test_host_slice_calls_from_many_threads():
    """The crate's functions are Sync (concurrent calls legal); host-slice calls
    from several threads give the same bits as the same calls made serially."""
    import threading
    shapes = [(2, 100, 130, 64, True), (1, 257, 257, 128, False), (3, 33, 500, 32, False), (1, 1000, 700, 96, True)]
    inputs = []
    for i, (bh, sq, sk, d, causal) in enumerate(shapes * 2):
        inputs.append((bh, sq, sk, d, causal, random_vec(bh * sq * d, 10 + i), random_vec(bh * sk * d, 20 + i),
                       random_vec(bh * sk * d, 30 + i)))
    serial = []
    for bh, sq, sk, d, causal, q, k, v in inputs:
        out = np.zeros(bh * sq * d, np.float32)
        fa.flash_attention_multihead_v3(q, k, v, 1, bh, sq, sk, d, fa.FlashAttentionConfig(causal=causal), out)
        serial.append(out)
    results = [None] * len(inputs)
    errors = []

    def work(i):
        try:
            bh, sq, sk, d, causal, q, k, v = inputs[i]
            for _ in range(3):
                out = np.zeros(bh * sq * d, np.float32)
                fa.flash_attention_multihead_v3(q, k, v, 1, bh, sq, sk, d, fa.FlashAttentionConfig(causal=causal), out)
                if results[i] is not None and not np.array_equal(results[i], out):
                    errors.append(f"thread {i}: calls disagree")
                results[i] = out
        except Exception as e:   # pragma: no cover - reported below
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(inputs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
    for i, out in enumerate(results):
        assert np.array_equal(out, serial[i]), i


def test_host_slice_staged_calls_from_many_threads():
    """Up to four host-slice calls per device run at once, each with its own
    stream, device staging buffer and pinned ring (further callers wait for a
    free one).  Six threads of calls large enough for the pinned ring, f32
    and bf16 mixed, each repeated: every output equals the device API's on
    the same inputs, bit for bit."""
    import threading
    torch = _torch()
    dev = torch.device("cuda", 0)
    shapes = [(8, 2048, 2048, 128, True), (3, 4000, 1500, 100, False), (16, 1000, 1000, 64, True),
              (1, 3, 300001, 24, False), (6, 1500, 4096, 128, False), (4, 2048, 2048, 128, True)]
    cases = []
    for i, (bh, sq, sk, d, causal) in enumerate(shapes):
        q, k, v = random_vec(bh * sq * d, 90 + i), random_vec(bh * sk * d, 100 + i), random_vec(bh * sk * d, 110 + i)
        lp = i % 3 == 2 and d % 8 == 0
        if lp:
            q16, k16, v16 = (fa.f32_to_bf16_bits(a) for a in (q, k, v))
            t = [torch.from_numpy(a.view(np.int16)).to(dev) for a in (q16, k16, v16)]
            out = torch.zeros(bh * sq * d, device=dev)
            fa.attention_device_lp(fa.DTYPE_BF16, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), 1, bh, sq, sk,
                                   d, causal, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            cases.append((bh, sq, sk, d, causal, (q16, k16, v16), True, out.cpu().numpy()))
        else:
            cases.append((bh, sq, sk, d, causal, (q, k, v), False, _device_run(3, q, k, v, bh, sq, sk, d, causal)))
    errors = []

    def work(i):
        try:
            bh, sq, sk, d, causal, (q, k, v), lp, want = cases[i]
            cfg = fa.FlashAttentionConfig(causal=causal)
            for rep in range(3):
                out = np.full(bh * sq * d, 7.0, np.float32)
                if lp:
                    fa.flash_attention_multihead_lp(fa.DTYPE_BF16, q, k, v, 1, bh, sq, sk, d, cfg, out)
                else:
                    fa.flash_attention_multihead_v3(q, k, v, 1, bh, sq, sk, d, cfg, out)
                if not np.array_equal(out, want):
                    errors.append(f"thread {i} call {rep}: differs from the device API")
        except Exception as e:   # pragma: no cover - reported below
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=180)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors


def test_host_slices_staged_copies_match_device_api():
    """Host slices move through a ring of 16 MiB pinned buffers, 4 deep; the
    sizes here put segment ends inside chunks, odd byte counts (16-bit inputs),
    an upload that wraps the ring (K/V of 36 MB each), a download of several
    chunks (O of 18 MB) and copies under and over the 1 MiB threading cut.
    The host-slice call runs the same kernels on the same data as the device
    call, so the outputs agree bit for bit."""
    cases = [(3, 1111, 30001, 100, False), (5, 9001, 300, 100, True), (1, 7, 5, 3, False),
             (32, 2048, 2048, 128, True), (5, 16384, 512, 128, False)]
    for i, (bh, sq, sk, d, causal) in enumerate(cases):
        q, k, v = random_vec(bh * sq * d, 40 + i), random_vec(bh * sk * d, 50 + i), random_vec(bh * sk * d, 60 + i)
        host = np.full(bh * sq * d, 7.0, np.float32)
        fa.flash_attention_multihead_v2(q, k, v, 1, bh, sq, sk, d, fa.FlashAttentionConfig(causal=causal), host)
        dev = _device_run(2, q, k, v, bh, sq, sk, d, causal)
        assert np.array_equal(host, dev), (bh, sq, sk, d, causal)
    # 16-bit inputs: an odd number of elements per tensor, a K/V upload over
    # several chunks; config 2 in bf16.
    torch = _torch()
    dev = torch.device("cuda", 0)
    for i, (bh, sq, sk, d, causal) in enumerate([(1, 3, 4194305, 3, False), (32, 2048, 2048, 128, True)]):
        q16 = fa.f32_to_bf16_bits(random_vec(bh * sq * d, 70 + i))
        k16 = fa.f32_to_bf16_bits(random_vec(bh * sk * d, 72 + i))
        v16 = fa.f32_to_bf16_bits(random_vec(bh * sk * d, 74 + i))
        host = np.full(bh * sq * d, 7.0, np.float32)
        fa.flash_attention_multihead_lp(fa.DTYPE_BF16, q16, k16, v16, 1, bh, sq, sk, d,
                                        fa.FlashAttentionConfig(causal=causal), host)
        t16 = [torch.from_numpy(a.view(np.int16)).to(dev) for a in (q16, k16, v16)]
        out = torch.zeros(bh * sq * d, device=dev)
        fa.attention_device_lp(fa.DTYPE_BF16, t16[0].data_ptr(), t16[1].data_ptr(), t16[2].data_ptr(), 1, bh, sq, sk,
                               d, causal, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(host, out.cpu().numpy()), (bh, sq, sk, d, causal)


def test_host_slices_odd_16bit_counts_copy_every_byte():
    """K and V of 15969 x 33 bf16 values are 1053954 bytes each (256m + 2):
    the copy pool splits them over four threads, and every byte must reach the
    device.  A first call with other values leaves different bytes in the
    pinned ring, so a piece the partition skipped would show as a stale last
    element (the large last K / V values make that visible) and the host-slice
    output would differ from the device API's."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    bh, sq, sk, d = 1, 64, 15969, 33
    q16 = fa.f32_to_bf16_bits(random_vec(bh * sq * d, 81))
    k = random_vec(bh * sk * d, 82)
    v = random_vec(bh * sk * d, 83)
    k[-1], v[-1] = 6.0, 40.0
    k16, v16 = fa.f32_to_bf16_bits(k), fa.f32_to_bf16_bits(v)
    junk = np.full(bh * sq * d, 7.0, np.float32)
    fa.flash_attention_multihead_lp(fa.DTYPE_BF16, q16, fa.f32_to_bf16_bits(-k), fa.f32_to_bf16_bits(-v), 1, bh,
                                    sq, sk, d, None, junk)
    host = np.full(bh * sq * d, 7.0, np.float32)
    fa.flash_attention_multihead_lp(fa.DTYPE_BF16, q16, k16, v16, 1, bh, sq, sk, d, None, host)
    t16 = [torch.from_numpy(a.view(np.int16)).to(dev) for a in (q16, k16, v16)]
    out = torch.zeros(bh * sq * d, device=dev)
    fa.attention_device_lp(fa.DTYPE_BF16, t16[0].data_ptr(), t16[1].data_ptr(), t16[2].data_ptr(), 1, bh, sq, sk,
                           d, False, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(host, out.cpu().numpy())
    assert not np.array_equal(host, junk)


def test_split_workspace_per_stream_and_graph_replay():
    """Split partials live in a workspace kept per stream: calls queued on two
    streams without synchronising in between must not share it, a later call
    that needs a larger workspace must not disturb earlier queued ones, and a
    captured graph of a decode call stays valid across replays (each replay
    checked, with eager calls on other shapes between replays)."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(93)

    def make(bh, sq, sk, d):
        q = rng.standard_normal(bh * sq * d, dtype=np.float32)
        k = rng.standard_normal(bh * sk * d, dtype=np.float32)
        v = rng.standard_normal(bh * sk * d, dtype=np.float32)
        t = [torch.from_numpy(a).to(dev) for a in (q, k, v)]
        return (bh, sq, sk, d), (q, k, v), t, torch.zeros(bh * sq * d, device=dev)

    small = [make(4, 1, 3000, 128), make(2, 16, 2000, 64), make(3, 3, 1500, 128)]
    big = make(32, 1, 8192, 128)   # needs a larger workspace than any of the above
    want = {}
    for case in small + [big]:
        (bh, sq, sk, d), (q, k, v), _, _ = case
        want[id(case)] = cpu_v2(q, k, v, bh, sq, sk, d, False)

    def queue(case, stream):
        (bh, sq, sk, d), _, (tq, tk, tv), out = case
        fa.attention_device(2, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, bh, sq, sk, d, False,
                            out.data_ptr(), stream.cuda_stream)

    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for rep in range(3):
        for i, case in enumerate(small):
            queue(case, s1 if (i + rep) % 2 == 0 else s2)
        queue(big, s1)              # grows s1's workspace while earlier calls may still run
        queue(small[rep], s1)
        torch.cuda.synchronize()
        for case in small + [big]:
            assert_parity(case[3].cpu().numpy(), want[id(case)], f"stream rep {rep} {case[0]}")

    # graph capture of a decode call (workspace created before capture)
    case = small[0]
    gs = torch.cuda.Stream()
    queue(case, gs)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gs):
        queue(case, gs)
    for rep in range(4):
        case[3].fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(case[3].cpu().numpy(), want[id(case)], f"graph replay {rep}")
        queue(small[1 + rep % 2], gs)   # eager work on the capture stream between replays
        queue(big, torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert_parity(small[1 + rep % 2][3].cpu().numpy(), want[id(small[1 + rep % 2])], f"eager after replay {rep}")


def test_release_stream_workspace_returns_device_memory():
    """A split call keeps its partials in a workspace per stream; releasing it
    gives the memory back.  Forced split-KV with 128 key splits over 64 heads
    of 64 queries at d64: about 138 MB of partials per stream.  Each of six
    streams gets a call, its output (bit-identical to the same call on the
    default stream), a check that the device lost at least the workspace,
    the release, and a check that the memory came back."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    bh, sq, sk, d, splits = 64, 64, 8192, 64, 128
    s = fa.describe_launch(2, 1, bh, sq, sk, d, False, fa.PATH_SPLITKV, splits)
    ws = int(s.split("workspace=")[1])
    assert 100e6 < ws < 256 << 20, s
    rng = np.random.default_rng(77)
    t = [torch.from_numpy(rng.standard_normal(n, dtype=np.float32)).to(dev) for n in (bh * sq * d, bh * sk * d,
                                                                                      bh * sk * d)]
    out = torch.zeros(bh * sq * d, device=dev)

    def call(stream):
        fa.attention_device(2, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), 1, bh, sq, sk, d, False,
                            out.data_ptr(), stream, path=fa.PATH_SPLITKV, num_splits=splits)

    call(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = out.cpu().numpy().copy()
    for i in range(6):
        st = torch.cuda.Stream()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        out.zero_()
        torch.cuda.synchronize()
        call(st.cuda_stream)
        st.synchronize()
        assert np.array_equal(out.cpu().numpy(), want), i
        free1 = torch.cuda.mem_get_info()[0]
        fa.release_stream_workspace(st.cuda_stream)
        free2 = torch.cuda.mem_get_info()[0]
        print(f"[workspace] stream {i}: free before {free0 / 2**20:.0f} MiB, with workspace "
              f"{free1 / 2**20:.0f} MiB, after release {free2 / 2**20:.0f} MiB", flush=True)
        assert free0 - free1 >= ws, (free0, free1, ws)
        assert abs(free2 - free0) < 16 << 20, (free0, free2)
    fa.release_stream_workspace(torch.cuda.current_stream().cuda_stream)
    fa.release_stream_workspace(torch.cuda.current_stream().cuda_stream)   # nothing kept: still FA_OK


def test_requests_beyond_device_memory_fail_cleanly():
    """FA_ERR_ALLOC before anything is queued, out untouched, the library
    usable afterwards: (a) naive attention on device pointers whose score
    matrix (2^19 x 2^19 f32 = 1 TiB) exceeds the device; (b) a forced split
    of 32 heads x 16384 queries x 1024 key splits at d256 (551 GB of
    partials)."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    n, d = 1 << 19, 2050
    q = torch.zeros(n * d, device=dev)
    out = torch.full((n * d,), 5.0, device=dev)
    with pytest.raises(fa.FaError) as e:
        fa.naive_device(q.data_ptr(), q.data_ptr(), q.data_ptr(), 1, 1, n, n, d, False, out.data_ptr(),
                        torch.cuda.current_stream().cuda_stream)
    assert e.value.status == fa.FA_ERR_ALLOC
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())
    del q, out
    bh, sq, sk, d = 32, 16384, 65536, 256
    s = fa.describe_launch(2, 1, bh, sq, sk, d, False, fa.PATH_SPLITKV, 1024)
    assert int(s.split("workspace=")[1]) > 400e9, s
    q = torch.zeros(bh * sq * d, device=dev)
    kv = torch.zeros(bh * sk * d, device=dev)
    out = torch.full((bh * sq * d,), 5.0, device=dev)
    with pytest.raises(fa.FaError) as e:
        fa.attention_device(2, q.data_ptr(), kv.data_ptr(), kv.data_ptr(), 1, bh, sq, sk, d, False, out.data_ptr(),
                            torch.cuda.current_stream().cuda_stream, path=fa.PATH_SPLITKV, num_splits=1024)
    assert e.value.status == fa.FA_ERR_ALLOC
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())
    del q, kv, out
    torch.cuda.empty_cache()
    q = random_vec(64 * 32, 5)
    want = cpu_v2(q, q, q, 1, 64, 64, 32, True)
    got = _device_run(2, q, q, q, 1, 64, 64, 32, True)
    assert_parity(got, want, "after FA_ERR_ALLOC")


def test_captured_calls_own_their_workspace():
    """A split call captured into a graph takes its stream's workspace over,
    so replays never share partials with later eager calls on the capture
    stream.  Two graphs are captured on one stream (an eager call before each
    capture makes the buffer the capture takes), then replayed on two other
    streams while an eager split call of a third shape runs on the capture
    stream, with no synchronisation between them; every output must match
    its reference, on every repetition."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(94)

    def make(bh, sq, sk, d):
        arrs = [rng.standard_normal(n, dtype=np.float32) for n in (bh * sq * d, bh * sk * d, bh * sk * d)]
        t = [torch.from_numpy(a).to(dev) for a in arrs]
        return (bh, sq, sk, d), arrs, t, torch.zeros(bh * sq * d, device=dev)

    cases = [make(4, 1, 3000, 128), make(2, 16, 2000, 64), make(3, 3, 1500, 128)]
    want = [cpu_v2(*c[1], *c[0], False) for c in cases]

    def queue(case, stream):
        (bh, sq, sk, d), _, (tq, tk, tv), out = case
        fa.attention_device(2, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, bh, sq, sk, d, False,
                            out.data_ptr(), stream.cuda_stream)

    gs, r1, r2 = torch.cuda.Stream(), torch.cuda.Stream(), torch.cuda.Stream()
    graphs = []
    for case in cases[:2]:
        queue(case, gs)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=gs):
            queue(case, gs)
        graphs.append(g)
    torch.cuda.synchronize()
    for rep in range(4):
        for c in cases:
            c[3].fill_(7.0)
        torch.cuda.synchronize()
        with torch.cuda.stream(r1):
            graphs[0].replay()
        with torch.cuda.stream(r2):
            graphs[1].replay()
        queue(cases[2], gs)
        torch.cuda.synchronize()
        for i, c in enumerate(cases):
            assert_parity(c[3].cpu().numpy(), want[i], f"rep {rep} case {i}")
    fa.release_stream_workspace(gs.cuda_stream)
