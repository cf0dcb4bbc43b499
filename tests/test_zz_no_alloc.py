"""The allocation-free entry point fa_device_ex_noalloc against fa_device_ex.

fa_device_ex_noalloc takes the same arguments and runs the same kernels as
fa_device_ex, with the split partials in the library's device-global scratch
array instead of a hipMalloc'd workspace.  Each case makes two calls in a
row, the second on a smaller input (the scratch keeps the first call's
partials; nothing may depend on them), and checks both against
fa_device_ex's output on the same inputs: the same kernels on the same data
give the same bits, and the north_star bar (max-abs 2e-5, relative L2 1e-5)
is asserted as well.  Every case here runs a split plan, so the scratch is
used; plans that need more than the array holds are refused untouched.
"""
from __future__ import annotations

import re

import numpy as np
import pytest

import flash_attention_amd as fa
from fa_testutil import assert_parity

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def _torch():
    import torch
    return torch


def _tensors(bh, sq, sk, d, seed):
    torch = _torch()
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(bh * sq * d, dtype=np.float32)
    k = rng.standard_normal(bh * sk * d, dtype=np.float32)
    v = rng.standard_normal(bh * sk * d, dtype=np.float32)
    return [torch.from_numpy(a).to(dev) for a in (q, k, v)]


def _call(fn, variant, t, bh, sq, sk, d, causal, path, splits):
    torch = _torch()
    out = torch.full((bh * sq * d,), 7.0, device=t[0].device)
    fn(variant, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), 1, bh, sq, sk, d, causal, out.data_ptr(),
       torch.cuda.current_stream().cuda_stream, path=path, num_splits=splits)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _workspace(variant, bh, sq, sk, d, causal, path, splits):
    s = fa.describe_launch(variant, 1, bh, sq, sk, d, causal, path, splits)
    m = re.search(r"workspace=(\d+)", s)
    assert m, f"not a split plan: {s}"
    return int(m.group(1))


# (variant, bh, sq, sk, d, causal, path, splits): first a larger call, then a smaller one
PAIRS = [
    # row-streaming split-KV decode
    ((2, 16, 1, 20000, 128, False, fa.PATH_AUTO, 0), (3, 4, 1, 3000, 128, False, fa.PATH_AUTO, 0)),
    # 16-row split-KV tiles
    ((3, 8, 16, 8192, 128, False, fa.PATH_AUTO, 0), (2, 2, 5, 900, 64, True, fa.PATH_SPLITKV, 3)),
    # prefill key split: the 16-head 1000 x 1000 d256 causal shape (48 MiB of partials)
    ((3, 16, 1000, 1000, 256, True, fa.PATH_AUTO, 0), (2, 2, 300, 700, 64, False, fa.PATH_PREFILL, 3)),
    # key split of the column-group kernels for heads wider than 256
    ((3, 4, 300, 2000, 1024, False, fa.PATH_PREFILL, 4), (2, 2, 100, 700, 512, True, fa.PATH_PREFILL, 3)),
]


def test_noalloc_allocates_nothing_on_a_fresh_stream():
    """Two no-alloc calls (a 48 MiB key-split plan, then a smaller one) on a
    stream no fa_device_ex call has used leave the device's free memory
    exactly as it was; the same plan through fa_device_ex on another fresh
    stream does allocate its workspace (the positive control).  Inputs and
    outputs are allocated, and each stream's first use (torch fills on it)
    made, before the free memory is read."""
    torch = _torch()
    fa.init()
    cases = [PAIRS[2][0], PAIRS[2][1]]
    data = []
    for i, (variant, bh, sq, sk, d, causal, path, splits) in enumerate(cases):
        t = _tensors(bh, sq, sk, d, 600 + i)
        data.append((t, torch.empty(bh * sq * d, device=t[0].device), torch.empty(bh * sq * d, device=t[0].device)))
    torch.cuda.synchronize()

    def run(fn, stream, which):
        for (variant, bh, sq, sk, d, causal, path, splits), (t, o_na, o_ex) in zip(cases, data):
            out = o_na if which == "na" else o_ex
            fn(variant, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), 1, bh, sq, sk, d, causal, out.data_ptr(),
               stream.cuda_stream, path=path, num_splits=splits)
        stream.synchronize()

    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for s in (s1, s2):
        with torch.cuda.stream(s):
            for _t, o_na, o_ex in data:
                o_na.fill_(7.0)
                o_ex.fill_(7.0)
        s.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    run(fa.attention_device_noalloc, s1, "na")
    free1 = torch.cuda.mem_get_info()[0]
    print(f"[no-alloc] free device memory {free0} -> {free1} across two no-alloc calls", flush=True)
    assert free1 == free0
    ws = _workspace(*cases[0])
    run(fa.attention_device, s2, "ex")
    free2 = torch.cuda.mem_get_info()[0]
    print(f"[no-alloc] fa_device_ex on a fresh stream: free {free1} -> {free2} (workspace {ws})", flush=True)
    assert free1 - free2 >= ws
    fa.release_stream_workspace(s2.cuda_stream)
    for (_t, o_na, o_ex), case in zip(data, cases):
        assert np.array_equal(o_na.cpu().numpy(), o_ex.cpu().numpy()), case


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_fa_device_ex_on_two_calls(first, second):
    fa.init()
    for i, case in enumerate((first, second)):
        variant, bh, sq, sk, d, causal, path, splits = case
        what = f"call {i + 1}: v{variant} bh={bh} sq={sq} sk={sk} d={d} causal={causal} path={path} splits={splits}"
        print(f"[no-alloc] {what}", flush=True)
        ws = _workspace(variant, bh, sq, sk, d, causal, path, splits)
        assert 0 < ws <= SCRATCH_BYTES, (what, ws)
        t = _tensors(bh, sq, sk, d, 500 + i)
        want = _call(fa.attention_device, variant, t, bh, sq, sk, d, causal, path, splits)
        got = _call(fa.attention_device_noalloc, variant, t, bh, sq, sk, d, causal, path, splits)
        assert_parity(got, want, what)
        assert np.array_equal(got, want), what


def test_noalloc_refuses_plans_beyond_the_scratch():
    """4 heads x 1024 queries in 16-row tiles x 32 forced key splits at d256:
    8192 partials of 16.5 KB = 135 MB > 64 MiB, refused before any launch."""
    fa.init()
    bh, sq, sk, d = 4, 1024, 2048, 256
    ws = _workspace(2, bh, sq, sk, d, False, fa.PATH_SPLITKV, 32)
    assert ws > SCRATCH_BYTES
    t = _tensors(bh, sq, sk, d, 9)
    with pytest.raises(fa.FaError) as e:
        _call(fa.attention_device_noalloc, 2, t, bh, sq, sk, d, False, fa.PATH_SPLITKV, 32)
    assert e.value.status == fa.FA_ERR_SCRATCH


def test_noalloc_heads_wider_than_2048_need_no_scratch():
    """Heads wider than 2048 columns accumulate O in the output rows: the
    no-alloc entry point runs them as fa_device_ex does, bit for bit."""
    fa.init()
    bh, sq, sk, d = 2, 40, 70, 2050
    assert "workspace=" not in fa.describe_launch(2, 1, bh, sq, sk, d, True)
    t = _tensors(bh, sq, sk, d, 10)
    want = _call(fa.attention_device, 2, t, bh, sq, sk, d, True, fa.PATH_AUTO, 0)
    got = _call(fa.attention_device_noalloc, 2, t, bh, sq, sk, d, True, fa.PATH_AUTO, 0)
    assert np.array_equal(got, want)


def test_noalloc_prefill_without_split_needs_no_scratch():
    """A full-grid prefill (no split) runs through the no-alloc entry point as
    through fa_device_ex."""
    fa.init()
    bh, sq, sk, d = 32, 2048, 2048, 64
    assert "workspace=" not in fa.describe_launch(3, 1, bh, sq, sk, d, True)
    t = _tensors(bh, sq, sk, d, 11)
    want = _call(fa.attention_device, 3, t, bh, sq, sk, d, True, fa.PATH_AUTO, 0)
    got = _call(fa.attention_device_noalloc, 3, t, bh, sq, sk, d, True, fa.PATH_AUTO, 0)
    assert np.array_equal(got, want)
