"""Host-side checks of the C ABI (libfa_hip.so) that need no GPU.

* the library loads and exports every function include/fa_hip.h declares;
* the crate's shape asserts (src/common.rs:51-54, :87-90) map to status
  codes in the same order (q, k, v, out), checked before any device access;
* zero-sized dims return FA_OK and leave out untouched (src/common.rs:56,
  tests/correctness.rs:465-504);
* without a visible device every compute entry point fails loudly with
  FA_ERR_NO_DEVICE (no CPU fallback exists);
* launch planning (fa_describe_launch): kernel choice per d_head, load path,
  split-KV for short queries, v1's own split instantiations, unsupported d_head.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import flash_attention_amd as fa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fa_hip.h")


def _has_gpu() -> bool:
    return os.path.exists("/dev/kfd")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 16
    lib = fa.lib()
    for name in names:
        assert hasattr(lib, name), f"{name} declared in fa_hip.h but not exported"
    assert sorted(fa.EXPORTED_SYMBOLS) == names
    out = subprocess.run(["nm", "-D", "--defined-only", fa.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (fa_[a-z0-9_]+)$", out, flags=re.M))
    assert exported == set(names)


def test_product_library_does_not_link_the_oracle():
    out = subprocess.run(["ldd", fa.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "oracle" not in out
    dyn = subprocess.run(["nm", "-D", fa.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "oracle_" not in dyn


def test_status_strings():
    assert fa.status_string(fa.FA_OK) == "ok"
    assert fa.status_string(fa.FA_ERR_Q_SHAPE) == "q shape mismatch"
    assert fa.status_string(fa.FA_ERR_K_SHAPE) == "k shape mismatch"
    assert fa.status_string(fa.FA_ERR_V_SHAPE) == "v shape mismatch"
    assert fa.status_string(fa.FA_ERR_OUT_SHAPE) == "out shape mismatch"
    for code in range(5, 13):
        assert fa.status_string(code) not in ("ok", "unknown status")
    assert fa.status_string(999) == "unknown status"


def test_config_default_mirrors_reference():
    c = fa.lib().fa_config_default()
    assert (c.block_size_q, c.block_size_kv, c.causal) == (64, 128, 0)   # src/common.rs:28-36


@pytest.mark.parametrize("variant", (1, 2, 3))
def test_shape_mismatch_order_and_messages(variant):
    f = fa.VARIANTS[variant]
    sq, sk, d = 4, 4, 8
    q = np.zeros(sq * d, np.float32)
    k = np.zeros(sk * d, np.float32)
    v = np.zeros(sk * d, np.float32)
    cfg = fa.FlashAttentionConfig()
    # every operand wrong: q is reported first, as check_shapes asserts q first
    with pytest.raises(fa.ShapeMismatch, match="^q shape mismatch$"):
        f(q[:-1], k[:-1], v[:-1], sq, sk, d, cfg, np.zeros(sq * d - 1, np.float32))
    with pytest.raises(fa.ShapeMismatch, match="^k shape mismatch$"):
        f(q, k[:-1], v[:-1], sq, sk, d, cfg, np.zeros(sq * d - 1, np.float32))
    with pytest.raises(fa.ShapeMismatch, match="^v shape mismatch$"):
        f(q, k, v[:-1], sq, sk, d, cfg, np.zeros(sq * d - 1, np.float32))
    with pytest.raises(fa.ShapeMismatch, match="^out shape mismatch$"):
        f(q, k, v, sq, sk, d, cfg, np.zeros(sq * d - 1, np.float32))
    # the ShapeMismatch is also an AssertionError, as the crate's assert_eq! panics
    with pytest.raises(AssertionError):
        f(q[:-1], k, v, sq, sk, d, cfg, np.zeros(sq * d, np.float32))


@pytest.mark.parametrize("variant", (1, 2, 3))
def test_multihead_shape_mismatch(variant):
    f = fa.MULTIHEAD_VARIANTS[variant]
    b, h, sq, sk, d = 2, 2, 4, 4, 8
    q = np.zeros(b * h * sq * d, np.float32)
    k = np.zeros(b * h * sk * d, np.float32)
    with pytest.raises(fa.ShapeMismatch, match="q shape"):
        f(q[:-1], k, k, b, h, sq, sk, d, None, np.zeros(b * h * sq * d, np.float32))
    with pytest.raises(fa.ShapeMismatch, match="out shape"):
        f(q, k, k, b, h, sq, sk, d, None, np.zeros(b * h * sq * d + 1, np.float32))


@pytest.mark.parametrize("variant", (1, 2, 3))
def test_zero_sized_dims_leave_out_untouched_without_device(variant):
    f = fa.VARIANTS[variant]
    d = 8
    out = np.full(4 * d, 12.5, np.float32)
    f(np.ones(4 * d, np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32), 4, 0, d, None, out)
    assert np.all(out == 12.5)
    f(np.zeros(0, np.float32), np.ones(4 * d, np.float32), np.ones(4 * d, np.float32), 0, 4, d, None,
      np.zeros(0, np.float32))
    f(np.zeros(0, np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32), 4, 4, 0, None,
      np.zeros(0, np.float32))
    m = fa.MULTIHEAD_VARIANTS[variant]
    out = np.full(0, 12.5, np.float32)
    m(np.zeros(0, np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32), 0, 3, 4, 4, d, None, out)


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_no_device_fails_loudly():
    with pytest.raises(fa.FaError) as e:
        fa.init()
    assert e.value.status == fa.FA_ERR_NO_DEVICE
    d = 16
    out = np.full(8 * d, 7.0, np.float32)
    for variant in (1, 2, 3):
        with pytest.raises(fa.FaError) as e:
            fa.VARIANTS[variant](np.ones(8 * d, np.float32), np.ones(8 * d, np.float32),
                                 np.ones(8 * d, np.float32), 8, 8, d, None, out)
        assert e.value.status == fa.FA_ERR_NO_DEVICE
        assert np.all(out == 7.0)
    with pytest.raises(fa.FaError) as e:
        fa.attention_device(2, 16, 16, 16, 1, 1, 8, 8, d, False, 16)
    assert e.value.status == fa.FA_ERR_NO_DEVICE
    with pytest.raises(fa.FaError) as e:
        fa.naive_attention(np.ones(8 * d, np.float32), np.ones(8 * d, np.float32), np.ones(8 * d, np.float32),
                           8, 8, d, True, out)
    assert e.value.status == fa.FA_ERR_NO_DEVICE and np.all(out == 7.0)


def test_naive_shape_checks_without_device():
    d = 4
    q, k, v, o = (np.ones(n * d, np.float32) for n in (3, 5, 5, 3))
    bad = np.ones(2, np.float32)
    for args, status in [((bad, k, v, o), fa.FA_ERR_Q_SHAPE), ((q, bad, v, o), fa.FA_ERR_K_SHAPE),
                         ((q, k, bad, o), fa.FA_ERR_V_SHAPE), ((q, k, v, bad), fa.FA_ERR_OUT_SHAPE),
                         ((bad, bad, bad, bad), fa.FA_ERR_Q_SHAPE)]:
        with pytest.raises(fa.ShapeMismatch) as e:
            fa.naive_attention(args[0], args[1], args[2], 3, 5, d, False, args[3])
        assert e.value.status == status
    # seq_len_q == 0 or d_head == 0: nothing to compute, no device needed
    fa.naive_attention(np.zeros(0, np.float32), k, v, 0, 5, d, False, np.zeros(0, np.float32))
    fa.naive_attention(*(np.zeros(0, np.float32),) * 3, 3, 5, 0, False, np.zeros(0, np.float32))
    with pytest.raises(fa.FaError) as e:   # bad precision is rejected before any device work
        fa.naive_device(16, 16, 16, 1, 1, 3, 5, d, False, 16, 0, 7)
    assert e.value.status in (fa.FA_ERR_INVALID_ARG, fa.FA_ERR_NO_DEVICE)


def test_bad_code_object_path_fails_with_module_or_no_device():
    code = ("import sys; sys.path.insert(0, %r); import flash_attention_amd as fa\n"
            "try:\n    fa.init(); print('ok')\nexcept fa.FaError as e:\n    print(e.status)\n"
            % os.path.join(ROOT, "flash-attention-cpu_amd"))
    env = dict(os.environ, FA_HIP_MODULE="/nonexistent/fa_kernels.hsaco")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                         timeout=120).stdout.strip()
    expect = fa.FA_ERR_MODULE if _has_gpu() else fa.FA_ERR_NO_DEVICE
    assert out == str(expect)


def describe(variant, b, h, sq, sk, d, causal, path=fa.PATH_AUTO, splits=0, dtype=fa.DTYPE_F32):
    return fa.describe_launch(variant, b, h, sq, sk, d, causal, path, splits, dtype)


def test_planning_prefill_kernels():
    # v3 pairs query blocks nqb-1-r and r when the pairs fill whole rounds (256 CUs)
    assert describe(3, 1, 32, 2048, 2048, 128, True) == "fa_prefill_v3_d128_2 grid=256x1x1 block=512 two_blocks"
    assert describe(3, 1, 8, 16384, 16384, 128, True).endswith("grid=512x1x1 block=512 two_blocks")
    assert describe(3, 1, 16, 2048, 2048, 128, True) == "fa_prefill_v3_d128_2 grid=256x1x1 block=512"   # 128 pairs
    assert describe(3, 1, 32, 2048, 2048, 120, True) == "fa_prefill_v3_d128_2 grid=512x1x1 block=512"   # d < D
    assert describe(3, 1, 32, 1920, 2048, 128, True) == "fa_prefill_v3_d128_2 grid=480x1x1 block=512"   # nqb odd
    assert describe(2, 1, 32, 2048, 2048, 128, True).startswith("fa_prefill_v2_d128_1 grid=512x1x1")
    assert describe(1, 1, 32, 2048, 2048, 128, True).startswith("fa_prefill_v1_d128_1")
    assert describe(2, 1, 8, 16384, 16384, 128, True).startswith("fa_prefill_v2_d128_1 grid=1024x1x1")
    assert describe(2, 1, 16, 4096, 1024, 256, False).startswith("fa_prefill_v2_d256_1")
    assert describe(2, 1, 1, 256, 256, 64, False, fa.PATH_PREFILL).startswith("fa_prefill_v2_d64_1 grid=2x1x1")
    for d, pad in ((1, 32), (17, 32), (33, 64), (65, 128), (129, 256), (256, 256)):
        loader = 1 if d % 4 == 0 else 0
        assert describe(2, 1, 1, 100, 100, d, False).startswith(f"fa_prefill_v2_d{pad}_{loader}"), d
    assert describe(3, 1, 1, 100, 100, 17, False).startswith("fa_prefill_v3_d32_0")
    assert describe(3, 1, 1, 100, 100, 40, False).startswith("fa_prefill_v3_d64_2")


def test_planning_split_kv():
    # seq_q <= 4: the row-streaming decode (whole-row K/V loads)
    s = describe(2, 1, 32, 1, 32768, 128, False)
    assert s.startswith("fa_decode_rows_d128_q1 grid=512x1x1 block=256") and "fa_merge_d128 grid=8x1x1 block=256" in s
    assert "splits=16 split_len=2048" in s
    assert describe(3, 1, 32, 2, 32768, 64, False).startswith("fa_decode_rows_d64_q2 grid=512x1x1")
    assert describe(2, 1, 8, 4, 9000, 256, True).startswith("fa_decode_rows_d256_q4")
    assert describe(2, 1, 8, 5, 9000, 256, False).startswith("fa_decode_d256_1")   # 5 rows: 16-row tiles
    assert describe(2, 1, 8, 1, 9000, 18, False).startswith("fa_decode_d32_0")     # d % 4 != 0: tiles
    s = describe(2, 1, 32, 1, 32768, 128, False, fa.PATH_SPLITKV)                  # forced 16-row tiles
    assert s.startswith("fa_decode_d128_2 grid=256x1x1") and "splits=8 split_len=4096" in s    # one per CU
    assert describe(2, 1, 4, 3, 100, 64, False, fa.PATH_SPLITKV_ROWS, 2).startswith("fa_decode_rows_d64_q4 grid=8x1x1")
    for bad in ((2, 1, 4, 5, 1000, 64), (2, 1, 4, 1, 1000, 18)):   # seq_q > 4; d % 4 != 0
        with pytest.raises(fa.FaError) as e:
            describe(*bad, False, fa.PATH_SPLITKV_ROWS)
        assert e.value.status == fa.FA_ERR_UNSUPPORTED
    # 16-bit: seq_q = 1 and d % 8 == 0 with D >= 64 only
    assert describe(2, 1, 32, 1, 32768, 128, False, dtype=fa.DTYPE_BF16).startswith("fa_decode_rows_bf16_d128_q1")
    assert describe(2, 1, 32, 1, 32768, 256, False, dtype=fa.DTYPE_F16).startswith("fa_decode_rows_f16_d256_q1")
    assert describe(2, 1, 32, 2, 32768, 128, False, dtype=fa.DTYPE_BF16).startswith("fa_prefill_lp_bf16")
    # v1 takes split-KV too, on its own instantiations (per-block normalisation, no causal skip)
    assert describe(1, 1, 4, 1, 1000, 64, False, fa.PATH_SPLITKV_ROWS).startswith("fa_decode_rows_v1_d64_q1 grid=12x1x1")
    assert "fa_decode" in describe(3, 1, 32, 16, 32768, 128, False)
    assert describe(1, 1, 32, 16, 32768, 128, False).startswith("fa_decode_v1_d128_2 grid=256x1x1")      # config 4b
    s = describe(1, 1, 32, 1, 32768, 128, False)                                                          # config 4a
    assert s.startswith("fa_decode_rows_v1_d128_q1 grid=512x1x1") and "fa_merge_d128 grid=8x1x1" in s
    assert describe(1, 1, 1, 256, 256, 64, False) == "fa_decode_v1_d64_2 grid=16x1x1 block=256"          # config 1
    assert describe(1, 1, 8, 5, 9000, 128, True, fa.PATH_SPLITKV, 0).startswith("fa_decode_v1_d128_2 ")
    assert describe(1, 1, 8, 5, 9000, 200, True, fa.PATH_SPLITKV, 0).startswith("fa_decode_v1_d256_1 ")
    assert describe(1, 1, 8, 5, 9000, 126, True, fa.PATH_SPLITKV, 0).startswith("fa_decode_v1_d128_0 ")
    assert "fa_decode" in describe(2, 1, 32, 16, 200, 128, False)         # short keys too
    assert describe(2, 1, 512, 1, 64, 128, False) == "fa_decode_rows_d128_q1 grid=512x1x1 block=256"
    assert "fa_decode" not in describe(2, 1, 32, 33, 200, 128, False)     # three tiles, short keys: prefill
    assert "fa_decode" not in describe(2, 1, 32, 16, 32768, 128, False, fa.PATH_PREFILL)
    s = describe(2, 1, 1, 40, 300, 64, True, fa.PATH_SPLITKV, 3)
    assert s.startswith("fa_decode_d64_2 grid=9x1x1") and "splits=3 split_len=128" in s
    # decode steps (<= 32 queries) take split-KV whatever the grid; one split
    # writes its rows directly (no workspace, no merge)
    assert describe(2, 1, 512, 1, 1024, 128, False) == "fa_decode_rows_d128_q1 grid=512x1x1 block=256"
    # the split-KV grid is one-dimensional: any number of slices (up to 2^31 workgroups)
    assert describe(2, 1, 70000, 1, 64, 32, False) == "fa_decode_rows_d32_q1 grid=70000x1x1 block=256"
    assert describe(2, 1, 70000, 20, 300, 64, False) == "fa_decode_d64_2 grid=140000x1x1 block=256"
    assert describe(2, 1, 256, 1, 4096, 128, False).startswith("fa_decode_rows_d128_q1 grid=512x1x1")
    assert describe(2, 1, 256, 32, 2048, 128, False) == "fa_decode_d128_2 grid=512x1x1 block=256"
    assert describe(2, 1, 256, 16, 1024, 256, False) == "fa_decode_d256_1 grid=256x1x1 block=256"
    assert describe(2, 1, 256, 64, 4096, 128, False).startswith("fa_prefill_v2_d128_1 ")   # 4 tiles: prefill
    assert describe(3, 1, 512, 1, 1024, 128, False, dtype=fa.DTYPE_BF16).startswith(
        "fa_decode_rows_bf16_d128_q1 grid=512x1x1")
    assert describe(3, 1, 256, 16, 2048, 128, False, dtype=fa.DTYPE_BF16).startswith("fa_prefill_lp_bf16")
    # tiles of decode steps one per CU, at least 256 keys per split
    assert "splits=4 split_len=1024" in describe(2, 1, 64, 16, 4096, 128, False)
    assert "splits=32 split_len=256" in describe(2, 1, 1, 1, 8192, 128, False)
    # small f32 prefills (grid below the CU count, <= 128 tiles x heads, >= 256 keys): 16-row tiles
    assert describe(2, 1, 1, 256, 256, 64, False) == "fa_decode_d64_2 grid=16x1x1 block=256"   # config 1
    assert describe(3, 1, 1, 2048, 2048, 128, True).startswith("fa_decode_d128_2 grid=512x1x1")
    assert describe(3, 1, 2, 2048, 2048, 128, True).startswith("fa_prefill_v3_d128_2")   # 256 tiles x heads
    assert describe(3, 1, 1, 200, 200, 64, False).startswith("fa_prefill_v3_d64_2")      # fewer than 256 keys
    assert describe(3, 1, 1, 256, 256, 64, False, dtype=fa.DTYPE_BF16).startswith("fa_prefill_lp_bf16")


def test_planning_stream_split_prefill():
    # config 5c: 8 query blocks x 16 heads = 128 workgroups < 256 CUs; v3's
    # 16-key stages: blocks of 8, 16, ..., 56 and 63 stages, 287 per head,
    # 4592 in all -> runs of 18 over 256 workgroups; block slots = 256 + 128 - 1
    # of 8 tiles x (16 x 256 + 32) floats
    s = describe(3, 1, 16, 1000, 1000, 256, True)
    # merged a workgroup per 16-row tile (16 slices x 63 tiles), a wave per 64 columns
    assert s.startswith("fa_prefill_v3_d256_2s grid=256x1x1 block=512; fa_merge_tiles_d256 grid=1008x1x1 block=256; ")
    assert "stream_per=18" in s and f"workspace={(256 + 128 - 1) * 8 * (16 * 256 + 32) * 4}" in s
    # v2's 32-key stages: 4 + 8 + ... + 28 + 32 = 144 per head -> runs of 9
    assert "grid=256x1x1" in describe(2, 1, 16, 1000, 1000, 256, True) and \
        "stream_per=9" in describe(2, 1, 16, 1000, 1000, 256, True)
    # forced: the workgroup count, at least 4 stages per run
    assert describe(3, 1, 16, 1000, 1000, 256, True, fa.PATH_STREAM, 100).startswith("fa_prefill_v3_d256_2s grid=100x1x1")
    assert "stream_per=46" in describe(3, 1, 16, 1000, 1000, 256, True, fa.PATH_STREAM, 100)
    assert "stream_per=4" in describe(2, 1, 1, 256, 256, 64, False, fa.PATH_STREAM)   # 4 stages: one run
    # 16-bit: two resident workgroups per CU at D <= 128
    assert describe(2, 1, 16, 1000, 1000, 64, True, fa.PATH_STREAM, dtype=fa.DTYPE_BF16).startswith(
        "fa_prefill_lp_bf16_d64_2_t1s grid=")


def test_planning_stream_split_refuses_unit_totals_past_32_bits():
    # 2 slices x 3,000,000^2 at d32 has about 2.2e9 key-stage units: the
    # kernel's 32-bit unit indices would wrap, so the forced stream split is
    # unsupported (planned on the CPU only; this shape never runs)
    with pytest.raises(fa.FaError) as e:
        describe(2, 1, 2, 3_000_000, 3_000_000, 32, False, fa.PATH_STREAM)
    assert e.value.status == fa.FA_ERR_UNSUPPORTED
    with pytest.raises(fa.FaError) as e:
        describe(2, 1, 2, 3_000_000, 3_000_000, 32, False, fa.PATH_STREAM, 1)
    assert e.value.status == fa.FA_ERR_UNSUPPORTED
    # a long causal slice well inside the limit (131,406 units) is planned
    s = describe(2, 1, 1, 46336, 46336, 32, True, fa.PATH_STREAM)
    assert s.startswith("fa_prefill_v2_d32_1s ")


def test_planning_key_split_prefill():
    # config 5c's shape, split forced over 3 workgroups per block
    s = describe(3, 1, 16, 1000, 1000, 256, True, fa.PATH_PREFILL, 3)
    assert s.startswith("fa_prefill_v3_d256_2s grid=") and "fa_merge_tiles_d256 grid=1008x1x1" in s   # split instantiation
    assert "stream_per" not in s
    nks, split_len = int(s.split("splits=")[1].split()[0]), int(s.split("split_len=")[1].split()[0])
    assert split_len % 16 == 0 and nks * split_len >= 1000 > (nks - 1) * split_len
    # compact grid: split y of every 128-row block whose causal key end passes y * split_len
    wgs = 16 * sum(1 for y in range(nks) for qb in range(8) if min(1000, 128 * (qb + 1)) > y * split_len)
    assert f"grid={wgs}x1x1" in s
    # v1 (config 5c): every block visits all 1000 keys = 32 stages of 32; two splits of 16 stages
    s = describe(1, 1, 16, 1000, 1000, 256, True)
    assert s.startswith("fa_prefill_v1_d256_1s grid=256x1x1 block=512; fa_merge_tiles_d256 grid=1008x1x1 ")
    assert "splits=2 split_len=512" in s and "stream_per" not in s
    s = describe(1, 1, 16, 1000, 1000, 256, True, fa.PATH_PREFILL, 3)   # forced: all 8 blocks in every split
    assert s.startswith("fa_prefill_v1_d256_1s grid=384x1x1") and "splits=3 split_len=352" in s
    s = describe(1, 1, 16, 1000, 1000, 256, True, fa.PATH_STREAM)        # 16 x 8 x 32 stages in 256 runs of 16
    assert s.startswith("fa_prefill_v1_d256_1s grid=256x1x1") and "stream_per=16" in s
    assert "fa_merge" not in describe(3, 1, 32, 2048, 2048, 128, True)    # full grid
    s = describe(2, 1, 1, 300, 700, 64, False, fa.PATH_PREFILL, 3)   # 11 stages of 64 keys -> 4 per split
    assert s.startswith("fa_prefill_v2_d64_1s grid=9x1x1") and "splits=3 split_len=256" in s
    assert "fa_merge_tiles_d64 grid=19x1x1 block=64" in s   # 19 tiles of 16 rows, one wave each
    # register-order partials at D = 64, 128, 256 only: D = 32 and 16-bit inputs merge by rows
    assert "fa_merge_d32 grid=75x1x1 block=256" in describe(2, 1, 1, 300, 700, 32, False, fa.PATH_PREFILL, 3)
    assert "fa_merge_tiles_d128 grid=19x1x1 block=128" in describe(3, 1, 1, 300, 700, 128, False, fa.PATH_PREFILL, 3)
    assert "fa_merge_d128 grid=75x1x1" in describe(3, 1, 1, 300, 700, 128, False, fa.PATH_PREFILL, 3,
                                                    dtype=fa.DTYPE_BF16)
    assert "splits=6 split_len=128" in describe(3, 1, 1, 300, 700, 64, False, fa.PATH_PREFILL, 6)


def test_planning_errors():
    # f32 heads of 257..2048 columns: the column-group flash kernels (forced
    # prefill and key splits too); split-KV and 16-bit inputs stop at 256
    assert describe(2, 1, 1, 10, 10, 257, False).startswith("fa_prefill_v2_d512_0 grid=1x1x1 block=512")
    assert describe(3, 1, 4, 1000, 1000, 512, True).startswith("fa_prefill_v3_d512_2s ")   # key split
    assert describe(3, 1, 4, 1000, 1000, 1024, True).startswith("fa_prefill_v3_d1024_2s ")   # K / V buffers alternate
    assert describe(1, 1, 1, 10, 10, 1000, False).startswith("fa_prefill_v1_d1024_1 ")
    assert describe(2, 1, 1, 10, 10, 300, False, fa.PATH_PREFILL).startswith("fa_prefill_v2_d512_1 ")
    s = describe(2, 1, 1, 100, 700, 512, False, fa.PATH_PREFILL, 3)
    assert s.startswith("fa_prefill_v2_d512_1s ") and "fa_merge_d512" in s and "splits=3" in s
    s = describe(3, 1, 1, 100, 700, 1024, False, fa.PATH_PREFILL, 3)
    assert s.startswith("fa_prefill_v3_d1024_2s ") and "fa_merge_d1024" in s
    for kw in ({"path": fa.PATH_SPLITKV}, {"path": fa.PATH_SPLITKV_ROWS}, {"dtype": fa.DTYPE_BF16}):
        with pytest.raises(fa.FaError) as e:
            describe(2, 1, 1, 10, 10, 257, False, **kw)
        assert e.value.status == fa.FA_ERR_UNSUPPORTED, kw
    # decode shapes at wide heads stay on the prefill kernels
    assert describe(2, 1, 32, 1, 32768, 512, False).startswith("fa_prefill_v2_d512_1s ")   # key split
    # 1025..2048 columns: D = 2048, 16-row workgroups of 8 column-group waves
    assert describe(2, 1, 1, 10, 10, 1025, False) == "fa_prefill_v2_d2048_0 grid=1x1x1 block=512"
    assert describe(3, 1, 2, 100, 100, 2048, True) == "fa_prefill_v3_d2048_1 grid=14x1x1 block=512"
    s = describe(1, 1, 1, 100, 700, 1536, True, fa.PATH_PREFILL, 3)   # v1 key split, all keys per block
    assert s.startswith("fa_prefill_v1_d2048_1s grid=21x1x1") and "fa_merge_d2048" in s and "splits=3" in s
    assert describe(2, 1, 1, 40, 300, 1536, True, fa.PATH_STREAM, 7).startswith("fa_prefill_v2_d2048_1s grid=")
    # wider than 2048: the any-width flash kernels, one 8-wave workgroup per
    # 16-row query tile and slice (no workspace); O in registers up to 4096
    # columns, in the output rows beyond; scalar loads unless d % 4 == 0
    assert describe(2, 1, 1, 10, 10, 2049, False) == "fa_prefill_v2_dreg_0 grid=1x1x1 block=512"
    assert describe(1, 2, 3, 100, 700, 4096, True) == "fa_prefill_v1_dreg_1 grid=42x1x1 block=512"
    assert describe(3, 1, 1, 33, 9, 2052, True, fa.PATH_PREFILL).startswith("fa_prefill_v3_dreg_1 grid=3x1x1")
    assert describe(2, 1, 1, 10, 10, 4097, False) == "fa_prefill_v2_dany_0 grid=1x1x1 block=512"
    assert describe(3, 1, 2, 40, 40, 10000, True).startswith("fa_prefill_v3_dany_1 grid=6x1x1")
    # forced splits and 16-bit inputs are refused
    for kw in ({"path": fa.PATH_STREAM}, {"path": fa.PATH_SPLITKV}, {"path": fa.PATH_SPLITKV_ROWS},
               {"path": fa.PATH_PREFILL, "splits": 3}, {"dtype": fa.DTYPE_BF16}):
        with pytest.raises(fa.FaError) as e:
            describe(2, 1, 1, 10, 10, 2049, False, **kw)
        assert e.value.status == fa.FA_ERR_UNSUPPORTED, kw
    assert describe(1, 1, 1, 10, 1000, 64, False, fa.PATH_SPLITKV).startswith("fa_decode_v1_d64_2 grid=3x1x1")
    with pytest.raises(fa.FaError) as e:
        describe(4, 1, 1, 10, 10, 64, False)
    assert e.value.status == fa.FA_ERR_INVALID_ARG
    assert describe(2, 0, 1, 10, 10, 64, False) == "none"


def test_device_entry_rejects_bad_variant_without_touching_device():
    with pytest.raises(fa.FaError) as e:
        fa.attention_device(7, 16, 16, 16, 1, 1, 8, 8, 16, False, 16)
    assert e.value.status == fa.FA_ERR_INVALID_ARG


def test_probe_launch_rejects_bad_arguments_without_touching_device():
    # argument checks come before any device or code-object access
    for kind, buf, nbytes in ((-1, 16, 1 << 20), (6, 16, 1 << 20), (0, 0, 1 << 20), (3, 8, 1 << 20), (5, 16, 16)):
        with pytest.raises(fa.FaError) as e:
            fa.probe_launch(kind, 0, buf, nbytes, 10)
        assert e.value.status == fa.FA_ERR_INVALID_ARG
    for iters in (0, (1 << 20) + 1, -1):   # MFMA probes: 1 .. 2^20 iterations
        with pytest.raises(fa.FaError) as e:
            fa.probe_launch(fa.PROBE_MFMA_F32_16X16X4, 0, 16, 1 << 20, iters)
        assert e.value.status == fa.FA_ERR_INVALID_ARG


def test_cpp_mirror_header_compiles(tmp_path):
    hdr = os.path.join(ROOT, "flash-attention-cpu_amd", "csrc", "flash_attention.hpp")
    src = tmp_path / "use.cpp"
    src.write_text('#include "%s"\nint main() { flash_attention::FlashAttentionConfig c; '
                   'return c.block_size_q == 64 ? 0 : 1; }\n' % hdr)
    subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", os.path.join(ROOT, "include"), str(src)],
                   check=True)


def test_bf16_conversion_helpers():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.14159, np.inf, -np.inf, 0.0, -0.0, 65504.0],
                 np.float32)
    bits = fa.f32_to_bf16_bits(x)
    back = fa.bf16_bits_to_f32(bits)
    # ties to even: 1 + 2^-8 -> 1, 1 + 3*2^-8 -> 1 + 2^-6; specials kept
    assert list(back[:3]) == [1.0, 1.0, 1.0 + 2 ** -6]
    assert back[3] == -2.5 and abs(back[4] - 3.14159) < 2 ** -7 * 4
    assert np.isposinf(back[5]) and np.isneginf(back[6]) and back[7] == 0.0 and np.signbit(back[8])
    assert np.isnan(fa.bf16_bits_to_f32(fa.f32_to_bf16_bits(np.array([np.nan], np.float32))))[0]
    r = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    assert np.array_equal(fa.f32_to_bf16_bits(fa.bf16_bits_to_f32(fa.f32_to_bf16_bits(r))), fa.f32_to_bf16_bits(r))
    assert np.max(np.abs(fa.bf16_bits_to_f32(fa.f32_to_bf16_bits(r)) - r) / np.abs(r)) <= 2 ** -8


def test_planning_16bit_inputs():
    s = describe(3, 1, 32, 2048, 2048, 128, True, dtype=fa.DTYPE_BF16)
    assert s.startswith("fa_prefill_lp_bf16_d128_2_t1 grid=512x1x1 block=512")   # one round, causal: 1 tile/wave
    # forced stream split: two resident two-tile workgroups per CU;
    # 32 heads x (2 + 4 + ... + 32) = 8704 stages of 64 keys -> 512 runs of 17
    s = describe(3, 1, 32, 2048, 2048, 128, True, fa.PATH_STREAM, dtype=fa.DTYPE_BF16)
    assert s.startswith("fa_prefill_lp_bf16_d128_2_t2s grid=512x1x1 block=256") and "stream_per=17" in s
    assert describe(3, 1, 32, 2048, 2048, 128, False, dtype=fa.DTYPE_BF16).startswith(
        "fa_prefill_lp_bf16_d128_2_t2 grid=512x1x1 block=256")
    assert describe(3, 1, 8, 16384, 16384, 128, True, dtype=fa.DTYPE_BF16).startswith("fa_prefill_lp_bf16_d128_2_t2 ")
    assert describe(3, 1, 16, 4096, 1024, 256, False, dtype=fa.DTYPE_BF16).startswith("fa_prefill_lp_bf16_d256_2_t1 ")
    assert describe(2, 1, 2, 100, 100, 40, False, dtype=fa.DTYPE_F16).startswith("fa_prefill_lp_f16_d64_2_t1")
    assert describe(2, 1, 2, 100, 100, 20, False, dtype=fa.DTYPE_F16).startswith("fa_prefill_lp_f16_d32_0_t1")
    s = describe(3, 1, 32, 1, 32768, 128, False, dtype=fa.DTYPE_BF16)   # AUTO, seq_q 1: row-streaming decode
    assert s.startswith("fa_decode_rows_bf16_d128_q1 grid=512x1x1") and "fa_merge_d128 grid=8x1x1" in s
    s = describe(3, 1, 32, 4, 32768, 128, False, dtype=fa.DTYPE_BF16)   # AUTO, seq_q 4: key-split 16-bit prefill
    assert s.startswith("fa_prefill_lp_bf16_d128_2_t2s ") and "fa_merge_d128 grid=32x1x1" in s
    s = describe(3, 1, 32, 1, 32768, 128, False, fa.PATH_SPLITKV, dtype=fa.DTYPE_BF16)   # split-KV, 16-bit loads
    assert s.startswith("fa_decode_bf16_d128_1 grid=256x1x1") and "fa_merge_d128 grid=8x1x1" in s
    assert describe(2, 1, 1, 4, 512, 64, False, fa.PATH_SPLITKV, dtype=fa.DTYPE_F16).startswith("fa_decode_f16_d64_1")
    assert describe(3, 1, 1, 4, 512, 62, False, fa.PATH_SPLITKV, dtype=fa.DTYPE_F16).startswith("fa_decode_f16_d64_0")
    with pytest.raises(fa.FaError) as e:
        describe(1, 1, 1, 4, 512, 64, False, fa.PATH_SPLITKV, dtype=fa.DTYPE_BF16)   # no 16-bit v1 kernels
    assert e.value.status == fa.FA_ERR_INVALID_ARG
    with pytest.raises(fa.FaError) as e:
        describe(3, 1, 1, 4, 512, 64, False, dtype=7)
    assert e.value.status == fa.FA_ERR_INVALID_ARG


def test_lp_host_slices_reject_wide_heads_before_copying():
    """fa_multihead_lp with d_head > 256 is refused right after the shape
    checks: no device access (so no FA_ERR_NO_DEVICE here), out untouched."""
    bh, sq, sk, d = 1, 3, 5, 300
    q = np.zeros(bh * sq * d, np.uint16)
    k = np.zeros(bh * sk * d, np.uint16)
    out = np.full(bh * sq * d, 3.0, np.float32)
    with pytest.raises(fa.FaError) as e:
        fa.flash_attention_multihead_lp(fa.DTYPE_BF16, q, k, k, 1, bh, sq, sk, d, None, out)
    assert e.value.status == fa.FA_ERR_UNSUPPORTED
    assert np.all(out == 3.0)
