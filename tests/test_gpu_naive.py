"""GPU naive attention (materialised scores) through the C ABI.

fa_naive_attention restates naive_attention (src/naive.rs:14-75) on the GPU;
fa_naive_device adds a multi-head, device-pointer form that can compute in
f64.  Checked here against the oracle's CPU naive (oracle/fa_oracle.c:
oracle_naive_f32 / oracle_naive_f64_rows), the reference's known answers,
and its zero-dimension conventions.  The f64 form then serves as the
full-size reference for the flash kernels at configs 3 and 5, where the CPU
oracle can only sample rows.
"""
from __future__ import annotations

import numpy as np
import pytest

import flash_attention_amd as fa
import oracle
from fa_testutil import assert_parity, max_abs_diff, normal_vec, random_vec, rel_l2, uniform_vec

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    fa.init()


def _torch():
    import torch
    return torch


def naive_gpu_device(q, k, v, bh, sq, sk, d, causal, precision, guard=64):
    """fa_naive_device on copies of q/k/v; sentinels around the output."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    tq, tk, tv = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (q, k, v))
    buf = torch.full((bh * sq * d + 2 * guard,), 12.5, device=dev)
    out = buf[guard:guard + bh * sq * d]
    fa.naive_device(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, bh, sq, sk, d, causal, out.data_ptr(),
                    torch.cuda.current_stream().cuda_stream, precision)
    torch.cuda.synchronize()
    host = buf.cpu().numpy()
    assert np.all(host[:guard] == 12.5) and np.all(host[-guard:] == 12.5), "write outside out"
    return host[guard:guard + bh * sq * d]


SHAPES = [(1, 1, 1, False), (7, 13, 5, True), (64, 64, 64, False), (65, 129, 17, True), (100, 37, 128, True),
          (37, 100, 256, False), (300, 300, 33, True), (129, 200, 200, False), (17, 1000, 96, False)]


@pytest.mark.parametrize("sq,sk,d,causal", SHAPES)
def test_naive_f32_matches_oracle(sq, sk, d, causal):
    q, k, v = random_vec(sq * d, 1), random_vec(sk * d, 2), random_vec(sk * d, 3)
    out = np.full(sq * d, 7.0, dtype=np.float32)
    fa.naive_attention(q, k, v, sq, sk, d, causal, out)
    what = f"naive f32 {sq}x{sk} d={d} causal={causal}"
    assert_parity(out, oracle.naive_f32(q, k, v, sq, sk, d, causal), what)
    assert max_abs_diff(out, oracle.naive_f64(q, k, v, sq, sk, d, causal)) < 2e-5, what


@pytest.mark.parametrize("sq,sk,d,causal", SHAPES)
def test_naive_f64_matches_oracle_f64(sq, sk, d, causal):
    bh = 3
    q, k, v = random_vec(bh * sq * d, 4), random_vec(bh * sk * d, 5), random_vec(bh * sk * d, 6)
    got = naive_gpu_device(q, k, v, bh, sq, sk, d, causal, fa.NAIVE_F64)
    for h in range(bh):
        sq_sl, sk_sl = slice(h * sq * d, (h + 1) * sq * d), slice(h * sk * d, (h + 1) * sk * d)
        want = oracle.naive_f64(q[sq_sl], k[sk_sl], v[sk_sl], sq, sk, d, causal)
        # both exact to f64 rounding; the GPU result is then rounded to f32
        assert max_abs_diff(got[sq_sl], want) < 1e-6, (h, sq, sk, d, causal)
    got32 = naive_gpu_device(q, k, v, bh, sq, sk, d, causal, fa.NAIVE_F32)
    assert max_abs_diff(got32, got) < 2e-5


def test_naive_known_answers():
    # causal row 0 attends only to key 0 (tests/correctness.rs:240-263)
    sq = sk = 50
    d = 24
    q, k, v = random_vec(sq * d, 1), random_vec(sk * d, 2), random_vec(sk * d, 3)
    out = np.zeros(sq * d, dtype=np.float32)
    fa.naive_attention(q, k, v, sq, sk, d, True, out)
    assert max_abs_diff(out[:d], v[:d]) < 1e-6
    # one key: every row is V[0]
    out1 = np.zeros(sq * d, dtype=np.float32)
    fa.naive_attention(q, k[:d], v[:d], sq, 1, d, False, out1)
    assert max_abs_diff(out1.reshape(sq, d), np.tile(v[:d], (sq, 1))) < 1e-6
    # Q = 0: uniform weights, so causal row i is the mean of V[0..=i]
    out0 = np.zeros(sq * d, dtype=np.float32)
    fa.naive_attention(np.zeros(sq * d, np.float32), k, v, sq, sk, d, True, out0)
    prefix = np.cumsum(v.reshape(sk, d).astype(np.float64), axis=0) / np.arange(1, sk + 1)[:, None]
    assert max_abs_diff(out0.reshape(sq, d), prefix) < 1e-5


def test_naive_zero_dims_and_shape_errors():
    d = 8
    q, k, v = random_vec(4 * d, 1), random_vec(5 * d, 2), random_vec(5 * d, 3)
    # seq_len_k == 0: the crate zero-fills every output row (src/naive.rs:64)
    out = np.full(4 * d, 3.0, dtype=np.float32)
    fa.naive_attention(q, np.zeros(0, np.float32), np.zeros(0, np.float32), 4, 0, d, False, out)
    assert np.all(out == 0.0)
    # seq_len_q == 0 / d_head == 0: nothing to write
    fa.naive_attention(np.zeros(0, np.float32), k, v, 0, 5, d, True, np.zeros(0, np.float32))
    fa.naive_attention(np.zeros(0, np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32), 4, 5, 0, False,
                       np.zeros(0, np.float32))
    # assert_eq! order: q, k, v, out (src/naive.rs:24-27)
    bad = np.zeros(3, np.float32)
    with pytest.raises(fa.ShapeMismatch, match="q shape"):
        fa.naive_attention(bad, bad, bad, 4, 5, d, False, bad)
    with pytest.raises(fa.ShapeMismatch, match="k shape"):
        fa.naive_attention(q, bad, bad, 4, 5, d, False, bad)
    with pytest.raises(fa.ShapeMismatch, match="v shape"):
        fa.naive_attention(q, k, bad, 4, 5, d, False, bad)
    with pytest.raises(fa.ShapeMismatch, match="out shape"):
        fa.naive_attention(q, k, v, 4, 5, d, False, bad)


def test_naive_multihead_device_matches_flash():
    bh, sq, sk, d = 6, 333, 517, 80
    q, k, v = normal_vec(bh * sq * d, 1), normal_vec(bh * sk * d, 2), normal_vec(bh * sk * d, 3)
    for causal in (False, True):
        ref = naive_gpu_device(q, k, v, bh, sq, sk, d, causal, fa.NAIVE_F64)
        want = oracle.run(2, q, k, v, bh, sq, sk, d, causal, 64, 128)
        assert_parity(ref, want, f"naive f64 vs cpu v2 causal={causal}")


def _flash_vs_naive_f64(bh, sq, sk, d, causal, q, k, v, variants=(1, 2, 3)):
    """Every row of the flash kernels against the f64 naive on the GPU."""
    torch = _torch()
    dev = torch.device("cuda", 0)
    tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    ref = torch.empty(bh * sq * d, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    fa.naive_device(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, bh, sq, sk, d, causal, ref.data_ptr(), st,
                    fa.NAIVE_F64)
    out = torch.empty(bh * sq * d, device=dev)
    worst = {}
    for variant in variants:
        out.fill_(12.5)
        fa.attention_device(variant, tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), 1, bh, sq, sk, d, causal,
                            out.data_ptr(), st)
        diff = (out - ref).abs().max().item()
        rl2 = ((out.double() - ref.double()).norm() / ref.double().norm()).item()
        print(f"[naive-f64] {bh}x{sq}x{sk} d={d} causal={causal} v{variant}: max-abs {diff:.3e} rel-l2 {rl2:.3e}",
              flush=True)
        worst[variant] = (diff, rl2)
        assert diff < 2e-5 and rl2 < 1e-5, (variant, diff, rl2)
    return worst


def test_config3_every_row_against_naive_f64():
    bh, s, d = 8, 16384, 128
    q, k, v = normal_vec(bh * s * d, 1), normal_vec(bh * s * d, 2), normal_vec(bh * s * d, 3)
    _flash_vs_naive_f64(bh, s, s, d, True, q, k, v)


def test_config5_every_row_against_naive_f64():
    bh, sq, sk, d = 16, 4096, 1024, 256
    q, k = normal_vec(bh * sq * d, 1, 3.0), normal_vec(bh * sk * d, 2, 3.0)
    v = uniform_vec(bh * sk * d, 3)
    _flash_vs_naive_f64(bh, sq, sk, d, False, q, k, v)
    s = 1000
    q, k = normal_vec(bh * s * d, 1, 3.0), normal_vec(bh * s * d, 2, 3.0)
    v = uniform_vec(bh * s * d, 3)
    _flash_vs_naive_f64(bh, s, s, d, True, q, k, v)


def test_heads_wider_than_2048_every_row_against_naive_f64():
    """The any-width flash kernels at the bench row's width, d = 4096, at a
    width with a ragged last 64-column chunk and d % 4 != 0 (d = 3001: scalar
    loads) -- O in registers -- and past 4096 (O accumulated in the output
    rows), causal and not, every row of every variant against the f64 naive
    on the GPU; keys end inside a 64-key stage."""
    for bh, sq, sk, d, causal in [(2, 300, 300, 4096, True), (1, 257, 130, 3001, False), (2, 200, 211, 3001, True),
                                  (1, 150, 160, 4500, True)]:
        q, k, v = normal_vec(bh * sq * d, 11), normal_vec(bh * sk * d, 12), normal_vec(bh * sk * d, 13)
        plan = fa.describe_launch(3, 1, bh, sq, sk, d, causal)
        assert plan.startswith("fa_prefill_v3_dreg_" if d <= 4096 else "fa_prefill_v3_dany_"), plan
        _flash_vs_naive_f64(bh, sq, sk, d, causal, q, k, v)
