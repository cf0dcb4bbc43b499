"""Tensors of more than 2^31 elements (8.6 GB of f32) through the device API.

The crate indexes its slices with usize (src/v2.rs:197-200, src/common.rs:
68-101), so a single head may be longer than any 32-bit element count.  The
kernels address rows as 64-bit offsets from each slice's base and stage K / V
through buffer resources based at the stage's first row; these tests put the
rows that matter past element 2^31 and compare with the oracle's CPU v2
(oracle/, the restatement of src/v2.rs:160-385):

* prefill: Q and O of 2^31 + 32768 elements (one head of 2^24 + 256 rows,
  d_head 128) against 64 keys, every variant and the bf16 path; sampled rows
  at the start, on both sides of element 2^31 and at the end (rows are
  independent without a causal mask);
* decode: K and V of 2^31 + 4736 elements (2^24 + 37 keys) for 1 and 16
  queries on the split-KV kernels.  Each query row's own key, placed past
  element 2^31, is a multiple of the query, so that key dominates the
  softmax and a wrong row offset shows as a wrong V row in the output.
"""
from __future__ import annotations

import numpy as np
import pytest

import flash_attention_amd as fa
import oracle
from fa_testutil import assert_parity, max_abs_diff, rel_l2

pytestmark = pytest.mark.gpu

D = 128
PREFILL_ROWS = (1 << 24) + 256      # Q / O: 2^31 + 32768 elements
PREFILL_KEYS = 64
DECODE_KEYS = (1 << 24) + 37        # K / V: 2^31 + 4736 elements
GUARD = 64


@pytest.fixture(scope="module", autouse=True)
def _device():
    fa.init()
    yield
    # hand the tens of GB these tests held back to the device for later tests
    _torch().cuda.empty_cache()


def _torch():
    import torch
    return torch


def _sample_rows(n: int) -> np.ndarray:
    """Row indices at the start, around element 2^31 (row 2^24) and at the end."""
    b = 1 << 24
    idx = np.concatenate([np.arange(0, 256), np.arange(b - 256, b + 256), np.arange(n - 256, n)])
    return idx[(idx >= 0) & (idx < n)]


def test_prefill_q_and_o_past_2_31_elements():
    torch = _torch()
    dev = torch.device("cuda", 0)
    sq, sk = PREFILL_ROWS, PREFILL_KEYS
    assert sq * D > 2 ** 31
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    q = torch.randn(sq * D, device=dev, generator=g)
    k = torch.randn(sk * D, device=dev, generator=g)
    v = torch.randn(sk * D, device=dev, generator=g)
    buf = torch.full((sq * D + 2 * GUARD,), 12.5, device=dev)
    out = buf[GUARD:GUARD + sq * D]
    stream = torch.cuda.current_stream().cuda_stream
    rows = _sample_rows(sq)
    ridx = torch.from_numpy(rows).to(dev)
    q_rows = q.view(sq, D)[ridx].cpu().numpy().ravel()
    k_host, v_host = k.cpu().numpy(), v.cpu().numpy()
    want = oracle.run(2, q_rows, k_host, v_host, 1, rows.size, sk, D, False)
    for variant in (1, 2, 3):
        plan = fa.describe_launch(variant, 1, 1, sq, sk, D, False)
        print(f"[case] large prefill v{variant} {sq}x{sk} d={D}: {plan}", flush=True)
        out.fill_(-3.0)
        fa.attention_device(variant, q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, 1, sq, sk, D, False,
                            out.data_ptr(), stream)
        torch.cuda.synchronize()
        got = out.view(sq, D)[ridx].cpu().numpy().ravel()
        assert_parity(got, want, f"large prefill v{variant}")
        assert bool((out.view(sq, D)[-1] != -3.0).all()), "last row not written"
        assert float(buf[:GUARD].min()) == 12.5 and float(buf[-GUARD:].max()) == 12.5, "write outside out"
    # bf16 inputs: the same rows against the oracle on the widened inputs,
    # within the rounding of the probabilities (u/(1-u) * max|V|, u = 2^-8;
    # tests/test_gpu_lp.py derives the bound)
    q16, k16, v16 = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    q16_rows = q16.view(sq, D)[ridx].float().cpu().numpy().ravel()
    k32, v32 = k16.float().cpu().numpy(), v16.float().cpu().numpy()
    want16 = oracle.run(2, q16_rows, k32, v32, 1, rows.size, sk, D, False)
    print(f"[case] large prefill bf16: {fa.describe_launch(2, 1, 1, sq, sk, D, False, dtype=fa.DTYPE_BF16)}",
          flush=True)
    out.fill_(-3.0)
    fa.attention_device_lp(fa.DTYPE_BF16, q16.data_ptr(), k16.data_ptr(), v16.data_ptr(), 1, 1, sq, sk, D, False,
                           out.data_ptr(), stream)
    torch.cuda.synchronize()
    got16 = out.view(sq, D)[ridx].cpu().numpy().ravel()
    u = 2.0 ** -8
    tol = u / (1.0 - u) * float(np.max(np.abs(v32))) + 2e-5
    ma, rl = max_abs_diff(got16, want16), rel_l2(got16, want16)
    print(f"[lp-parity] large prefill bf16: max-abs {ma:.3g} (bound {tol:.3g}) rel-L2 {rl:.3g}", flush=True)
    assert ma <= tol and rl <= 2.0 ** -8
    assert float(buf[:GUARD].min()) == 12.5 and float(buf[-GUARD:].max()) == 12.5, "write outside out"


def test_decode_k_and_v_past_2_31_elements():
    torch = _torch()
    dev = torch.device("cuda", 0)
    sk = DECODE_KEYS
    assert sk * D > 2 ** 31
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    nq = 16
    q = torch.randn(nq * D, device=dev, generator=g)
    k = torch.randn(sk * D, device=dev, generator=g)
    v = torch.randn(sk * D, device=dev, generator=g)
    # query i's own key past element 2^31: 4 q_i, a logit of 4 |q_i|^2 / sqrt(128)
    # (about 45) against logits of about 1 for the other keys
    own = (1 << 24) + 5 + 2 * np.arange(nq)
    k.view(sk, D)[torch.from_numpy(own).to(dev)] = 4.0 * q.view(nq, D)
    k_host, v_host, q_host = k.cpu().numpy(), v.cpu().numpy(), q.cpu().numpy()
    stream = torch.cuda.current_stream().cuda_stream
    for sq in (1, nq):
        want = oracle.run(2, q_host[:sq * D], k_host, v_host, 1, sq, sk, D, False)
        # the dominant key is really the one read
        assert max_abs_diff(want, v_host.reshape(sk, D)[own[:sq]].ravel()) < 1e-3
        buf = torch.full((sq * D + 2 * GUARD,), 12.5, device=dev)
        out = buf[GUARD:GUARD + sq * D]
        for variant in (1, 2, 3):
            plan = fa.describe_launch(variant, 1, 1, sq, sk, D, False)
            print(f"[case] large decode v{variant} {sq}x{sk} d={D}: {plan}", flush=True)
            out.fill_(-3.0)
            fa.attention_device(variant, q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, 1, sq, sk, D, False,
                                out.data_ptr(), stream)
            torch.cuda.synchronize()
            assert_parity(out.cpu().numpy(), want, f"large decode v{variant} sq={sq}")
            assert float(buf[:GUARD].min()) == 12.5 and float(buf[-GUARD:].max()) == 12.5, "write outside out"
