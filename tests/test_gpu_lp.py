"""GPU parity of the 16-bit-input path (fa_device_lp / fa_multihead_lp).

Reference: the oracle's CPU v2 (and the f64 GPU naive at full size) on the
same inputs widened to f32, which is exact.  The kernel's products are exact
and its sums f32; the one deliberate rounding is the probabilities p_j,
rounded to the input type (p^_j = p_j (1 + d_j), |d_j| <= u, u = 2^-8 bf16,
2^-11 f16) for the PV product, whose row sums l^ = sum_j p^_j come from the
same MFMA.  With w_j = p_j / l the output moves by
|sum_j w_j d_j (v_j - o)| / (1 + sum_j w_j d_j) <= u/(1-u) * sum_j w_j |v_j - o|
<= u/(1-u) * max|V| (o is the w-weighted mean of the v_j, and a mean absolute
deviation about the mean of values in [-M, M] is at most M).  The bar:
max-abs <= u/(1-u) * max|V| + 2e-5 and relative L2 <= u.  (f16 rounds
2^7 p_j, so |d_j| <= u holds down to p_j = 2^-21 of the row's reference;
below that the absolute error, at most 2^-32 per key against row sums of at
least 1, stays under the 2e-5 slack for rows of up to 85,000 such keys.)  Known answers that
involve no rounding (a row that sees one key returns that key's V row) are
checked bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import flash_attention_amd as fa
import oracle
from fa_testutil import attention_f64, long_row_f16_case, max_abs_diff, normal_vec, rel_l2, uniform_vec

pytestmark = pytest.mark.gpu

U = {fa.DTYPE_BF16: 2.0 ** -8, fa.DTYPE_F16: 2.0 ** -11}   # unit roundoff


def lp_bound(dtype, v32) -> float:
    """Max-abs bar: u/(1-u) * max|V| + 2e-5 (module docstring)."""
    u = U[dtype]
    return u / (1.0 - u) * float(np.max(np.abs(v32))) + 2e-5
NAME = {fa.DTYPE_BF16: "bf16", fa.DTYPE_F16: "f16"}


@pytest.fixture(scope="module", autouse=True)
def _device():
    fa.init()


def _torch():
    import torch
    return torch


def to16(x32: np.ndarray, dtype: int):
    """(16-bit array for the library, its exact f32 widening)."""
    if dtype == fa.DTYPE_BF16:
        bits = fa.f32_to_bf16_bits(x32)
        return bits, fa.bf16_bits_to_f32(bits)
    h = np.asarray(x32, dtype=np.float32).astype(np.float16)
    return h, h.astype(np.float32)


def lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, path=fa.PATH_AUTO, splits=0, guard=64, misalign=False,
              scale=None):
    """fa_device_lp on copies of the 16-bit inputs; sentinels around O."""
    torch = _torch()
    dev = torch.device("cuda", 0)

    def dev16(a):
        t = torch.from_numpy(a.view(np.int16).copy()).to(dev)
        if misalign:   # a 2-byte offset forces the register-staged loader
            buf = torch.zeros(a.size + 1, dtype=torch.int16, device=dev)
            buf[1:] = t
            return buf, buf[1:].data_ptr()
        return t, t.data_ptr()

    (tq, pq), (tk, pk), (tv, pv) = dev16(q16), dev16(k16), dev16(v16)
    buf = torch.full((bh * sq * d + 2 * guard,), 12.5, device=dev)
    out = buf[guard:guard + bh * sq * d]
    fa.attention_device_lp(dtype, pq, pk, pv, 1, bh, sq, sk, d, causal, out.data_ptr(),
                           torch.cuda.current_stream().cuda_stream, softmax_scale=scale, path=path, num_splits=splits)
    torch.cuda.synchronize()
    host = buf.cpu().numpy()
    assert np.all(host[:guard] == 12.5) and np.all(host[-guard:] == 12.5), "write outside out"
    return host[guard:guard + bh * sq * d]


def assert_lp(got, want, v32, dtype, what):
    u = U[dtype]
    tol = lp_bound(dtype, v32)
    ma, rl = max_abs_diff(got, want), rel_l2(got, want)
    print(f"[lp-parity] {what}: max-abs {ma:.3g} (bound {tol:.3g}) rel-L2 {rl:.3g} (bound {u:.3g})", flush=True)
    assert ma <= tol, (what, ma, tol)
    assert rl <= u, (what, rl, u)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_explicit_softmax_scale_on_every_path(dtype):
    """The explicit scale through the 16-bit prefill, its key split and
    stream split (D = 128) and the split-KV kernels (rows and tiles), against
    float64 attention on the widened inputs with Q * (s * sqrt(d)), under the
    derived bound."""
    rng = np.random.default_rng(97)
    A, P, K, S, T, R = fa.PATH_AUTO, fa.PATH_PREFILL, fa.PATH_PREFILL, fa.PATH_STREAM, fa.PATH_SPLITKV, fa.PATH_SPLITKV_ROWS
    cases = [((2, 300, 500, 64, True, 0.3), [(A, 0), (P, 0), (K, 3)]),
             ((1, 200, 700, 128, False, 0.05), [(A, 0), (P, 0), (K, 3), (S, 0)]),
             ((1, 130, 260, 256, True, 0.02), [(A, 0), (P, 0), (K, 2)]),
             ((4, 1, 3000, 128, False, 0.2), [(A, 0), (T, 4), (R, 4)]),
             ((2, 16, 1500, 64, False, 0.4), [(A, 0), (T, 3)])]
    for (bh, sq, sk, d, causal, scale), paths in cases:
        q16, q32 = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), dtype)
        k16, k32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        v16, v32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        qs = q32.astype(np.float64) * scale * np.sqrt(d)   # exact in float64
        want = np.concatenate([attention_f64(qs[h * sq * d:(h + 1) * sq * d], k32[h * sk * d:(h + 1) * sk * d],
                                             v32[h * sk * d:(h + 1) * sk * d], sq, sk, d, causal) for h in range(bh)])
        for path, splits in paths:
            what = (f"{NAME[dtype]} scale {scale} path={path} splits={splits} {bh}x{sq}x{sk} d={d} causal={causal}: "
                    f"{fa.describe_launch(3, 1, bh, sq, sk, d, causal, path, splits, dtype)}")
            print("[case]", what, flush=True)
            got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, path, splits, scale=scale)
            assert_lp(got, want, v32, dtype, what)


CASES = [(1, 1, 1, 8, False), (2, 64, 64, 64, False), (3, 100, 37, 128, True), (1, 37, 100, 256, False),
         (2, 300, 300, 32, True), (1, 129, 200, 96, False), (2, 257, 513, 128, True), (1, 700, 300, 64, True),
         (1, 17, 1000, 40, False), (2, 200, 200, 17, True), (1, 150, 90, 200, False), (1, 1000, 1000, 128, True)]


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_matches_oracle_on_widened_inputs(dtype):
    rng = np.random.default_rng(31)
    for bh, sq, sk, d, causal in CASES:
        q16, q32 = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), dtype)
        k16, k32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        v16, v32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        want = oracle.run(2, q32, k32, v32, bh, sq, sk, d, causal, 64, 128)
        what = f"{NAME[dtype]} {bh}x{sq}x{sk} d={d} causal={causal}"
        print("[case]", what, fa.describe_launch(3, 1, bh, sq, sk, d, causal, dtype=dtype), flush=True)
        got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal)
        assert_lp(got, want, v32, dtype, what)
        if d % 8 == 0:   # the register-staged loader on the same inputs
            got2 = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, misalign=True)
            assert_lp(got2, want, v32, dtype, what + " (misaligned)")


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_every_head_dim(dtype):
    rng = np.random.default_rng(5)
    for d in list(range(1, 33)) + [48, 63, 64, 65, 100, 127, 128, 129, 192, 255, 256]:
        bh, sq, sk = 1, 70, 90
        q16, q32 = to16(rng.uniform(-1, 1, bh * sq * d).astype(np.float32), dtype)
        k16, k32 = to16(rng.uniform(-1, 1, bh * sk * d).astype(np.float32), dtype)
        v16, v32 = to16(rng.uniform(-1, 1, bh * sk * d).astype(np.float32), dtype)
        for causal in (False, True):
            want = oracle.run(2, q32, k32, v32, bh, sq, sk, d, causal, 64, 128)
            got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal)
            assert_lp(got, want, v32, dtype, f"{NAME[dtype]} d={d} causal={causal}")


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_known_answers_are_exact(dtype):
    rng = np.random.default_rng(9)
    bh, s, d = 2, 300, 128
    q16, _ = to16(rng.standard_normal(bh * s * d, dtype=np.float32), dtype)
    k16, _ = to16(rng.standard_normal(bh * s * d, dtype=np.float32), dtype)
    v16, v32 = to16(rng.standard_normal(bh * s * d, dtype=np.float32), dtype)
    # causal row 0 sees only key 0: p = 1 exactly, O row 0 = V row 0 (tests/correctness.rs:240-263)
    out = lp_device(dtype, q16, k16, v16, bh, s, s, d, True).reshape(bh, s, d)
    for h in range(bh):
        assert np.array_equal(out[h, 0], v32.reshape(bh, s, d)[h, 0])
    # one key: every row is V[0]
    out1 = lp_device(dtype, q16, k16[:bh * d].copy(), v16[:bh * d].copy(), bh, s, 1, d, False).reshape(bh, s, d)
    for h in range(bh):   # head h's single key/value row is element block h of the first bh*d
        assert np.array_equal(out1[h], np.tile(v32[h * d:(h + 1) * d], (s, 1)))


def test_lp_f16_long_row_of_small_probabilities():
    """The f16 prefill on the long row of fa_testutil.long_row_f16_case, every
    key in one workgroup (forced prefill, no key split: a split not holding
    key 0 would take one of the small keys as its reference), against exact
    attention in float64 on the widened inputs, max-abs under u/(1-u) *
    max|V| + 2e-5 (O is near 0, so no relative bar).  Not against the CPU v2
    oracle: its f32 running sums add t ~ 179.5 ulp(1) once per key and round
    the same way every time, which leaves CPU v2 6.7e-4 off here."""
    q16, k16, v16, sq, sk, d = long_row_f16_case()
    q, k, v = (a.astype(np.float64).reshape(-1, d) for a in (q16, k16, v16))
    s = q @ k.T / 8.0                                  # scale 1/sqrt(64)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    want = ((p @ v) / p.sum(axis=1, keepdims=True)).ravel()
    print("[case] f16 long row", fa.describe_launch(3, 1, 1, sq, sk, d, False, fa.PATH_PREFILL, dtype=fa.DTYPE_F16),
          flush=True)
    got = lp_device(fa.DTYPE_F16, q16, k16, v16, 1, sq, sk, d, False, path=fa.PATH_PREFILL)
    tol = lp_bound(fa.DTYPE_F16, v16.astype(np.float32))
    ma = float(np.max(np.abs(got.astype(np.float64) - want)))
    print(f"[lp-parity] f16 long row: max-abs {ma:.3g} against float64 (bound {tol:.3g})", flush=True)
    assert ma <= tol, (ma, tol)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_key_split_and_determinism(dtype):
    rng = np.random.default_rng(12)
    for bh, sq, sk, d, causal in [(1, 1000, 1000, 256, True), (2, 300, 2000, 128, False), (3, 129, 1025, 64, True)]:
        q16, q32 = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), dtype)
        k16, k32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        v16, v32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        want = oracle.run(2, q32, k32, v32, bh, sq, sk, d, causal, 64, 128)
        for splits in (2, 5, 16):
            got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, fa.PATH_PREFILL, splits)
            assert_lp(got, want, v32, dtype, f"{NAME[dtype]} split={splits} {bh}x{sq}x{sk} d={d}")
        a = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal)
        b = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal)
        assert np.array_equal(a, b)
        assert_lp(a, want, v32, dtype, f"{NAME[dtype]} auto {bh}x{sq}x{sk} d={d}")


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_stream_split(dtype):
    """The stream split on the 16-bit kernels (FA_PATH_STREAM; AUTO does not
    choose it for 16-bit inputs): several workgroup counts at every head
    width, the two-tile kernel at d_head 65..128, and repeatable results."""
    rng = np.random.default_rng(13)
    for bh, sq, sk, d, causal in [(3, 1000, 1000, 128, True), (2, 300, 2000, 128, False), (3, 129, 1025, 64, True),
                                  (1, 700, 700, 256, True), (5, 77, 300, 32, True), (4, 600, 600, 100, True)]:
        q16, q32 = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), dtype)
        k16, k32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        v16, v32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        want = oracle.run(2, q32, k32, v32, bh, sq, sk, d, causal, 64, 128)
        for splits in (0, 3, 17, 200):
            plan = fa.describe_launch(3, 1, bh, sq, sk, d, causal, fa.PATH_STREAM, splits, dtype=dtype)
            assert "stream_per=" in plan, plan
            got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, fa.PATH_STREAM, splits)
            assert_lp(got, want, v32, dtype, f"{NAME[dtype]} stream {splits}: {plan}")
        if 64 < d <= 128:
            assert "_t2s " in fa.describe_launch(3, 1, bh, sq, sk, d, causal, fa.PATH_STREAM, dtype=dtype)
        a = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, fa.PATH_STREAM, 0)
        assert np.array_equal(a, lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, fa.PATH_STREAM, 0))


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_differential_fuzz(dtype):
    """Random shapes, paths and logit scales on the 16-bit prefill kernels
    (row sums on the PV MFMAs): d_head 1..256, ragged rows and keys, causal
    or not, automatic / forced prefill with key splits / stream split, logits
    up to sigma 4 per element (peaky rows dominated by one key), against the
    oracle's CPU v2 on the widened inputs under the derived bound."""
    rng = np.random.default_rng(2026)
    for case in range(24):
        d = int(rng.choice([1, 7, 32, 33, 64, 96, 127, 128, 160, 200, 256]))
        bh = int(rng.integers(1, 5))
        sq = int(rng.integers(1, 400))
        sk = int(rng.integers(1, 700))
        causal = bool(rng.integers(0, 2))
        sigma = float(rng.choice([0.5, 1.0, 2.0, 4.0]))
        path, splits = [(fa.PATH_AUTO, 0), (fa.PATH_PREFILL, 0), (fa.PATH_PREFILL, int(rng.integers(2, 9))),
                        (fa.PATH_STREAM, int(rng.integers(0, 40)))][int(rng.integers(0, 4))]
        if path == fa.PATH_STREAM and (sq < 2 or sq * bh < 2):
            path, splits = fa.PATH_AUTO, 0
        q16, q32 = to16((rng.standard_normal(bh * sq * d) * sigma).astype(np.float32), dtype)
        k16, k32 = to16((rng.standard_normal(bh * sk * d) * sigma).astype(np.float32), dtype)
        v16, v32 = to16(rng.uniform(-1, 1, bh * sk * d).astype(np.float32), dtype)
        try:
            plan = fa.describe_launch(3, 1, bh, sq, sk, d, causal, path, splits, dtype=dtype)
        except fa.FaError as e:   # e.g. a forced stream split the shape cannot take
            print(f"[fuzz] case {case}: {bh}x{sq}x{sk} d={d} path={path} splits={splits}: {e}", flush=True)
            continue
        what = f"{NAME[dtype]} fuzz {case}: {bh}x{sq}x{sk} d={d} causal={causal} sigma={sigma} {plan}"
        print("[case]", what, flush=True)
        want = oracle.run(2, q32, k32, v32, bh, sq, sk, d, causal, 64, 128)
        got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, path, splits)
        assert_lp(got, want, v32, dtype, what)


def test_lp_host_slices_shape_errors_and_zero_dims():
    dtype = fa.DTYPE_BF16
    rng = np.random.default_rng(2)
    bh, sq, sk, d = 2, 33, 65, 64
    q16, q32 = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), dtype)
    k16, k32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
    v16, v32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
    out = np.zeros(bh * sq * d, np.float32)
    fa.flash_attention_multihead_lp(dtype, q16, k16, v16, 1, bh, sq, sk, d, fa.FlashAttentionConfig(causal=True), out)
    assert_lp(out, oracle.run(2, q32, k32, v32, bh, sq, sk, d, True, 64, 128), v32, dtype, "host slices")
    f16q, _ = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), fa.DTYPE_F16)
    with pytest.raises(TypeError):
        fa.flash_attention_multihead_lp(dtype, f16q, k16, v16, 1, bh, sq, sk, d, None, out)
    for args, msg in [((q16[:-1], k16, v16, out), "q shape"), ((q16, k16[:-1], v16, out), "k shape"),
                      ((q16, k16, v16[:-1], out), "v shape"), ((q16, k16, v16, out[:-1]), "out shape")]:
        with pytest.raises(fa.ShapeMismatch, match=msg):
            fa.flash_attention_multihead_lp(dtype, args[0], args[1], args[2], 1, bh, sq, sk, d, None, args[3])
    keep = np.full(sq * d, 7.0, np.float32)
    fa.flash_attention_multihead_lp(dtype, q16[:sq * d], np.zeros(0, np.uint16), np.zeros(0, np.uint16), 1, 1, sq,
                                    0, d, None, keep)
    assert np.all(keep == 7.0)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_full_size_configs_against_naive_f64(dtype):
    """Configs 2 and 5 at full size, every row, against the f64 GPU naive on the widened inputs."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    for name, (bh, sq, sk, d, causal, sig, vu) in {"config2": (32, 2048, 2048, 128, True, 1.0, False),
                                                   "config5": (16, 4096, 1024, 256, False, 3.0, True)}.items():
        q16, q32 = to16(normal_vec(bh * sq * d, 1, sig), dtype)
        k16, k32 = to16(normal_vec(bh * sk * d, 2, sig), dtype)
        v16, v32 = to16(uniform_vec(bh * sk * d, 3) if vu else normal_vec(bh * sk * d, 3), dtype)
        tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q32, k32, v32))
        ref = torch.empty(bh * sq * d, device=dev)
        st = torch.cuda.current_stream().cuda_stream
        fa.naive_device(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, bh, sq, sk, d, causal, ref.data_ptr(), st,
                        fa.NAIVE_F64)
        del tq, tk, tv
        t16 = [torch.from_numpy(a.view(np.int16).copy()).to(dev) for a in (q16, k16, v16)]
        out = torch.full((bh * sq * d,), 12.5, device=dev)
        fa.attention_device_lp(dtype, t16[0].data_ptr(), t16[1].data_ptr(), t16[2].data_ptr(), 1, bh, sq, sk, d,
                               causal, out.data_ptr(), st)
        torch.cuda.synchronize()
        diff = (out - ref).abs().max().item()
        rl = ((out.double() - ref.double()).norm() / ref.double().norm()).item()
        tol = lp_bound(dtype, v32)
        print(f"[lp-naive-f64] {NAME[dtype]} {name}: max-abs {diff:.3g} (bound {tol:.3g}) rel-L2 {rl:.3g}",
              flush=True)
        assert diff <= tol and rl <= U[dtype], (name, diff, rl)


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_split_kv_decode_is_exact_widening(dtype):
    """The split-KV kernel (FA_PATH_SPLITKV) widens 16-bit loads to f32: no
    probability rounding, so the f32 bar applies against the oracle on the
    widened inputs.  AUTO takes the key-split 16-bit prefill (u bound)."""
    from fa_testutil import assert_parity
    rng = np.random.default_rng(40)
    cases = [(32, 1, 4096, 128, False), (4, 16, 2048, 128, False), (2, 5, 1000, 64, True), (3, 40, 777, 32, False),
             (1, 17, 3000, 256, False), (2, 1, 600, 60, False), (1, 33, 513, 37, True)]
    for bh, sq, sk, d, causal in cases:
        q16, q32 = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), dtype)
        k16, k32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        v16, v32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        want = oracle.run(2, q32, k32, v32, bh, sq, sk, d, causal, 64, 128)
        for path, splits in ((fa.PATH_AUTO, 0), (fa.PATH_SPLITKV, 0), (fa.PATH_SPLITKV, 3)):
            plan = fa.describe_launch(3, 1, bh, sq, sk, d, causal, path, splits, dtype)
            what = f"{NAME[dtype]} decode {bh}x{sq}x{sk} d={d} causal={causal} path={path} splits={splits}"
            print("[case]", what, plan, flush=True)
            got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, path, splits)
            if "fa_decode" in plan:
                assert_parity(got, want, what)
            else:
                assert_lp(got, want, v32, dtype, what)
        got = lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, fa.PATH_SPLITKV, 0, misalign=True)
        assert_parity(got, want, f"{NAME[dtype]} decode misaligned {bh}x{sq}x{sk} d={d}")


@pytest.mark.parametrize("dtype", [fa.DTYPE_BF16, fa.DTYPE_F16])
def test_lp_row_streaming_decode_is_exact_widening(dtype):
    """The row-streaming split-KV kernel (seq_q = 1, d % 8 == 0, d > 32)
    widens 16-byte chunks of 8 16-bit values exactly and computes in f32: the
    f32 bar against the oracle on the widened inputs.  Covers d below the
    padded size (lanes past d), ragged key ranges, splits whose waves get no
    keys, causal (only key 0 visible), and for f16 subnormal keys (scaled by
    2^-20, mostly below 2^-14), which the widening must keep."""
    from fa_testutil import assert_parity
    rng = np.random.default_rng(41)
    cases = [(32, 4096, 128, False, 1.0), (4, 777, 64, False, 1.0), (3, 1000, 256, False, 1.0),
             (2, 513, 72, True, 1.0), (5, 2000, 200, False, 1.0), (2, 40, 128, False, 1.0),
             (3, 1500, 128, False, 2.0 ** -20)]
    for bh, sk, d, causal, kscale in cases:
        sq = 1
        q16, q32 = to16(rng.standard_normal(bh * sq * d, dtype=np.float32), dtype)
        k16, k32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32) * np.float32(kscale), dtype)
        v16, v32 = to16(rng.standard_normal(bh * sk * d, dtype=np.float32), dtype)
        want = oracle.run(2, q32, k32, v32, bh, sq, sk, d, causal, 64, 128)
        for path, splits in ((fa.PATH_SPLITKV_ROWS, 0), (fa.PATH_SPLITKV_ROWS, 1), (fa.PATH_SPLITKV_ROWS, 3),
                             (fa.PATH_SPLITKV_ROWS, 40)):
            plan = fa.describe_launch(2, 1, bh, sq, sk, d, causal, path, splits, dtype)
            assert plan.startswith(f"fa_decode_rows_{NAME[dtype]}_"), plan
            what = f"{NAME[dtype]} rows {bh}x{sq}x{sk} d={d} causal={causal} kscale={kscale} splits={splits}"
            print("[case]", what, plan, flush=True)
            assert_parity(lp_device(dtype, q16, k16, v16, bh, sq, sk, d, causal, path, splits), want, what)
    # AUTO takes it for 16-bit decode steps; other shapes are refused on this path
    assert fa.describe_launch(2, 1, 32, 1, 32768, 128, False, dtype=dtype).startswith(
        f"fa_decode_rows_{NAME[dtype]}_d128_q1")
    for bad in ((2, 1, 4, 2, 1000, 128), (2, 1, 4, 1, 1000, 32), (2, 1, 4, 1, 1000, 100)):   # sq 2; D 32; d % 8
        with pytest.raises(fa.FaError):
            fa.describe_launch(*bad, False, fa.PATH_SPLITKV_ROWS, 0, dtype)
