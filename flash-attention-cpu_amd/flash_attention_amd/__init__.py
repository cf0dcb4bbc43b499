"""Python view of libfa_hip.so (the C ABI in include/fa_hip.h).

Mirrors the public API of the reference crate amaye15/flash-attention-cpu
(src/lib.rs:78-87) with the same names, argument order and meaning:

    flash_attention_v1/v2/v3(q, k, v, seq_len_q, seq_len_k, d_head, config, out)
    flash_attention_multihead_v1/v2/v3(q, k, v, batch, heads, seq_len_q,
                                       seq_len_k, d_head, config, out)
    flash_attention = flash_attention_v2
    flash_attention_multihead = flash_attention_multihead_v2
    FlashAttentionConfig(block_size_q=64, block_size_kv=128, causal=False)

``q``/``k``/``v`` are float32 buffers (numpy arrays) and ``out`` is written
in place, as ``&mut [f32]`` is in the crate.  Where the crate panics on a
shape mismatch (src/common.rs:51-54) these raise ``ShapeMismatch`` with the
same message.  All compute runs on the GPU; without a usable HIP device the
calls raise ``FaError`` -- there is no CPU fallback.

``attention_device`` is the device-resident form (raw device pointers and a
HIP stream, e.g. from torch tensors), used by the benchmark.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# FA_HIP_LIBRARY overrides the library (e.g. a build with other tuning macros);
# the code object is found next to it unless FA_HIP_MODULE names one.
LIB_PATH = os.environ.get("FA_HIP_LIBRARY") or os.path.join(_PKG_DIR, "libfa_hip.so")
MODULE_PATH = os.path.join(_PKG_DIR, "fa_kernels.hsaco")

FA_OK = 0
FA_ERR_Q_SHAPE = 1
FA_ERR_K_SHAPE = 2
FA_ERR_V_SHAPE = 3
FA_ERR_OUT_SHAPE = 4
FA_ERR_INVALID_ARG = 5
FA_ERR_UNSUPPORTED = 6
FA_ERR_NO_DEVICE = 7
FA_ERR_MODULE = 8
FA_ERR_ALLOC = 9
FA_ERR_LAUNCH = 10
FA_ERR_COPY = 11
FA_ERR_SCRATCH = 12

PATH_AUTO = 0
PATH_PREFILL = 1
PATH_SPLITKV = 2
PATH_SPLITKV_ROWS = 3
PATH_STREAM = 4

NAIVE_F32 = 0
NAIVE_F64 = 1

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

# Every symbol include/fa_hip.h declares.
EXPORTED_SYMBOLS = (
    "fa_status_string", "fa_config_default",
    "fa_v1", "fa_v2", "fa_v3", "fa_attention",
    "fa_multihead_v1", "fa_multihead_v2", "fa_multihead_v3", "fa_attention_multihead",
    "fa_device_v1", "fa_device_v2", "fa_device_v3", "fa_release_stream_workspace",
    "fa_device_ex", "fa_device_ex_noalloc",
    "fa_device_lp", "fa_multihead_lp",
    "fa_naive_attention", "fa_naive_device",
    "fa_init", "fa_describe_launch", "fa_probe_launch",
)


class FaError(RuntimeError):
    """A non-zero status from libfa_hip.so."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class ShapeMismatch(FaError, AssertionError):
    """The crate's shape assert (src/common.rs:51-54) failed."""


@dataclass
class FlashAttentionConfig:
    """FlashAttentionConfig (src/common.rs:16-36)."""

    block_size_q: int = 64
    block_size_kv: int = 128
    causal: bool = False


class _CConfig(ctypes.Structure):
    _fields_ = [("block_size_q", ctypes.c_size_t), ("block_size_kv", ctypes.c_size_t),
                ("causal", ctypes.c_uint8)]


class _COpts(ctypes.Structure):
    _fields_ = [("softmax_scale", ctypes.c_float), ("path", ctypes.c_int), ("num_splits", ctypes.c_int),
                ("dtype", ctypes.c_int)]


_lib = None
_F = ctypes.POINTER(ctypes.c_float)
_SZ = ctypes.c_size_t
_CFG = ctypes.POINTER(_CConfig)
_OPTS = ctypes.POINTER(_COpts)


def _share_hip_runtime_with_torch() -> None:
    """Load torch (if installed) before libfa_hip.so.

    PyTorch-ROCm wheels bundle their own libamdhip64 and resolve it by path;
    if libfa_hip.so pulled in /opt/rocm's copy first, a later ``import torch``
    would load a second HIP runtime and find no GPU.  Loaded the other way
    round, libfa_hip.so binds to torch's already-loaded libamdhip64.so.7 and
    the process has one runtime.  Set FA_NO_TORCH_PRELOAD=1 to skip."""
    if os.environ.get("FA_NO_TORCH_PRELOAD"):
        return
    try:
        import torch  # noqa: F401
    except Exception:   # torch absent or broken: nothing to share with
        pass


def lib() -> ctypes.CDLL:
    """Load libfa_hip.so (built by flash-attention-cpu_amd/build.py)."""
    global _lib
    if _lib is not None:
        return _lib
    _share_hip_runtime_with_torch()
    if not os.path.exists(LIB_PATH):
        raise FaError(FA_ERR_MODULE, f"{LIB_PATH} is not built; run flash-attention-cpu_amd/build.py")
    L = ctypes.CDLL(LIB_PATH)
    L.fa_status_string.restype = ctypes.c_char_p
    L.fa_status_string.argtypes = [ctypes.c_int]
    L.fa_config_default.restype = _CConfig
    single = [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _CFG, _F, _SZ]
    for name in ("fa_v1", "fa_v2", "fa_v3", "fa_attention"):
        getattr(L, name).argtypes = single
        getattr(L, name).restype = ctypes.c_int
    multi = [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _CFG, _F, _SZ]
    for name in ("fa_multihead_v1", "fa_multihead_v2", "fa_multihead_v3", "fa_attention_multihead"):
        getattr(L, name).argtypes = multi
        getattr(L, name).restype = ctypes.c_int
    dev = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _SZ, _SZ, _SZ, _SZ, _SZ,
           _CFG, ctypes.c_void_p]
    for name in ("fa_device_v1", "fa_device_v2", "fa_device_v3"):
        getattr(L, name).argtypes = dev
        getattr(L, name).restype = ctypes.c_int
    L.fa_release_stream_workspace.argtypes = [ctypes.c_void_p]
    L.fa_release_stream_workspace.restype = ctypes.c_int
    L.fa_device_ex.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                               ctypes.c_void_p, _SZ, _SZ, _SZ, _SZ, _SZ, _CFG, _OPTS, ctypes.c_void_p]
    L.fa_device_ex.restype = ctypes.c_int
    L.fa_device_ex_noalloc.argtypes = L.fa_device_ex.argtypes
    L.fa_device_ex_noalloc.restype = ctypes.c_int
    L.fa_device_lp.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                               _SZ, _SZ, _SZ, _SZ, _SZ, _CFG, _OPTS, ctypes.c_void_p]
    L.fa_device_lp.restype = ctypes.c_int
    L.fa_multihead_lp.argtypes = [ctypes.c_int, ctypes.c_void_p, _SZ, ctypes.c_void_p, _SZ, ctypes.c_void_p, _SZ,
                                  _SZ, _SZ, _SZ, _SZ, _SZ, _CFG, _F, _SZ]
    L.fa_multihead_lp.restype = ctypes.c_int
    L.fa_naive_attention.argtypes = [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, ctypes.c_int, _F, _SZ]
    L.fa_naive_attention.restype = ctypes.c_int
    L.fa_naive_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _SZ, _SZ,
                                  _SZ, _SZ, _SZ, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L.fa_naive_device.restype = ctypes.c_int
    L.fa_init.restype = ctypes.c_int
    L.fa_describe_launch.argtypes = [ctypes.c_int, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_int, _OPTS,
                                     ctypes.c_char_p, _SZ]
    L.fa_describe_launch.restype = ctypes.c_int
    L.fa_probe_launch.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, _SZ, ctypes.c_uint,
                                  ctypes.POINTER(ctypes.c_double)]
    L.fa_probe_launch.restype = ctypes.c_int
    _lib = L
    return L


def status_string(status: int) -> str:
    return lib().fa_status_string(int(status)).decode()


def _check(status: int) -> None:
    if status == FA_OK:
        return
    msg = status_string(status)
    if status in (FA_ERR_Q_SHAPE, FA_ERR_K_SHAPE, FA_ERR_V_SHAPE, FA_ERR_OUT_SHAPE):
        raise ShapeMismatch(status, msg)
    raise FaError(status, msg)


def _cfg(config: FlashAttentionConfig | None) -> _CConfig:
    if config is None:
        return lib().fa_config_default()
    return _CConfig(int(config.block_size_q), int(config.block_size_kv), 1 if config.causal else 0)


def _in(a) -> tuple[np.ndarray, int]:
    arr = np.ascontiguousarray(a, dtype=np.float32)
    return arr, arr.size


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_F) if a.size else None


def _out(out) -> np.ndarray:
    if not isinstance(out, np.ndarray) or out.dtype != np.float32 or not out.flags.c_contiguous:
        raise TypeError("out must be a C-contiguous numpy float32 array (written in place)")
    return out


def _single(name, q, k, v, seq_len_q, seq_len_k, d_head, config, out):
    q, nq = _in(q)
    k, nk = _in(k)
    v, nv = _in(v)
    out = _out(out)
    cfg = _cfg(config)
    _check(getattr(lib(), name)(_ptr(q), nq, _ptr(k), nk, _ptr(v), nv, seq_len_q, seq_len_k, d_head,
                                ctypes.byref(cfg), _ptr(out), out.size))


def _multi(name, q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out):
    q, nq = _in(q)
    k, nk = _in(k)
    v, nv = _in(v)
    out = _out(out)
    cfg = _cfg(config)
    _check(getattr(lib(), name)(_ptr(q), nq, _ptr(k), nk, _ptr(v), nv, batch, heads, seq_len_q, seq_len_k,
                                d_head, ctypes.byref(cfg), _ptr(out), out.size))


def flash_attention_v1(q, k, v, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention_v1 (src/v1.rs:51)."""
    _single("fa_v1", q, k, v, seq_len_q, seq_len_k, d_head, config, out)


def flash_attention_v2(q, k, v, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention_v2 (src/v2.rs:49)."""
    _single("fa_v2", q, k, v, seq_len_q, seq_len_k, d_head, config, out)


def flash_attention_v3(q, k, v, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention_v3 (src/v3.rs:61)."""
    _single("fa_v3", q, k, v, seq_len_q, seq_len_k, d_head, config, out)


def flash_attention_multihead_v1(q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention_multihead_v1 (src/v1.rs:134)."""
    _multi("fa_multihead_v1", q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out)


def flash_attention_multihead_v2(q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention_multihead_v2 (src/v2.rs:132)."""
    _multi("fa_multihead_v2", q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out)


def flash_attention_multihead_v3(q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention_multihead_v3 (src/v3.rs:144)."""
    _multi("fa_multihead_v3", q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out)


def flash_attention(q, k, v, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention (src/lib.rs:87): the v2 alias, through the C ABI's fa_attention."""
    _single("fa_attention", q, k, v, seq_len_q, seq_len_k, d_head, config, out)


def flash_attention_multihead(q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out) -> None:
    """flash_attention_multihead (src/lib.rs:86): the v2 alias, through fa_attention_multihead."""
    _multi("fa_attention_multihead", q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config, out)

VARIANTS = {1: flash_attention_v1, 2: flash_attention_v2, 3: flash_attention_v3}
MULTIHEAD_VARIANTS = {1: flash_attention_multihead_v1, 2: flash_attention_multihead_v2,
                      3: flash_attention_multihead_v3}


def f32_to_bf16_bits(x) -> np.ndarray:
    """Round f32 values to bfloat16 (nearest, ties to even); returns the 16-bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(bits) -> np.ndarray:
    """Widen bfloat16 patterns to f32 (exact)."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _in16(a, dtype: int) -> tuple[np.ndarray, int]:
    want = np.uint16 if dtype == DTYPE_BF16 else np.float16
    arr = np.ascontiguousarray(a)
    if arr.dtype != want:
        raise TypeError(f"16-bit inputs for dtype {dtype} must be numpy {np.dtype(want).name} "
                        "(bfloat16 as uint16 bit patterns)")
    return arr, arr.size


def flash_attention_multihead_lp(dtype: int, q, k, v, batch, heads, seq_len_q, seq_len_k, d_head, config,
                                 out) -> None:
    """16-bit Q/K/V (DTYPE_BF16: uint16 bit patterns, DTYPE_F16: float16), f32 out (fa_multihead_lp)."""
    q, nq = _in16(q, dtype)
    k, nk = _in16(k, dtype)
    v, nv = _in16(v, dtype)
    out = _out(out)
    cfg = _cfg(config)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p) if a.size else None   # noqa: E731
    _check(lib().fa_multihead_lp(int(dtype), ptr(q), nq, ptr(k), nk, ptr(v), nv, batch, heads, seq_len_q,
                                 seq_len_k, d_head, ctypes.byref(cfg), _ptr(out), out.size))


def attention_device_lp(dtype: int, q_ptr: int, k_ptr: int, v_ptr: int, batch: int, heads: int, seq_len_q: int,
                        seq_len_k: int, d_head: int, causal: bool, out_ptr: int, stream: int = 0,
                        softmax_scale: float | None = None, path: int = PATH_AUTO, num_splits: int = 0) -> None:
    """Queue a 16-bit-input call on device pointers (fa_device_lp); returns when queued."""
    cfg = _CConfig(64, 128, 1 if causal else 0)
    opts = _COpts(float(softmax_scale) if softmax_scale else 0.0, int(path), int(num_splits), int(dtype))
    _check(lib().fa_device_lp(int(dtype), ctypes.c_void_p(stream), ctypes.c_void_p(q_ptr), ctypes.c_void_p(k_ptr),
                              ctypes.c_void_p(v_ptr), batch, heads, seq_len_q, seq_len_k, d_head,
                              ctypes.byref(cfg), ctypes.byref(opts), ctypes.c_void_p(out_ptr)))


def naive_attention(q, k, v, seq_len_q, seq_len_k, d_head, causal, out) -> None:
    """naive_attention (src/naive.rs:14): materialised scores, on the GPU, f32."""
    q, nq = _in(q)
    k, nk = _in(k)
    v, nv = _in(v)
    out = _out(out)
    _check(lib().fa_naive_attention(_ptr(q), nq, _ptr(k), nk, _ptr(v), nv, seq_len_q, seq_len_k, d_head,
                                    1 if causal else 0, _ptr(out), out.size))


def naive_device(q_ptr: int, k_ptr: int, v_ptr: int, batch: int, heads: int, seq_len_q: int, seq_len_k: int,
                 d_head: int, causal: bool, out_ptr: int, stream: int = 0, precision: int = NAIVE_F32) -> None:
    """Queue naive attention on device pointers (fa_naive_device); NAIVE_F64 computes in f64."""
    _check(lib().fa_naive_device(ctypes.c_void_p(stream), ctypes.c_void_p(q_ptr), ctypes.c_void_p(k_ptr),
                                 ctypes.c_void_p(v_ptr), batch, heads, seq_len_q, seq_len_k, d_head,
                                 1 if causal else 0, int(precision), ctypes.c_void_p(out_ptr)))


def attention_device(variant: int, q_ptr: int, k_ptr: int, v_ptr: int, batch: int, heads: int,
                     seq_len_q: int, seq_len_k: int, d_head: int, causal: bool, out_ptr: int,
                     stream: int = 0, softmax_scale: float | None = None, path: int = PATH_AUTO,
                     num_splits: int = 0) -> None:
    """Queue one call on device pointers (fa_device_ex); returns when queued."""
    cfg = _CConfig(64, 128, 1 if causal else 0)
    opts = _COpts(float(softmax_scale) if softmax_scale else 0.0, int(path), int(num_splits))
    _check(lib().fa_device_ex(int(variant), ctypes.c_void_p(stream), ctypes.c_void_p(q_ptr),
                              ctypes.c_void_p(k_ptr), ctypes.c_void_p(v_ptr), batch, heads, seq_len_q,
                              seq_len_k, d_head, ctypes.byref(cfg), ctypes.byref(opts),
                              ctypes.c_void_p(out_ptr)))


def attention_device_noalloc(variant: int, q_ptr: int, k_ptr: int, v_ptr: int, batch: int, heads: int,
                             seq_len_q: int, seq_len_k: int, d_head: int, causal: bool, out_ptr: int,
                             stream: int = 0, softmax_scale: float | None = None, path: int = PATH_AUTO,
                             num_splits: int = 0) -> None:
    """As attention_device, through fa_device_ex_noalloc: split partials in the
    library's device-global scratch array, no device allocation."""
    cfg = _CConfig(64, 128, 1 if causal else 0)
    opts = _COpts(float(softmax_scale) if softmax_scale else 0.0, int(path), int(num_splits))
    _check(lib().fa_device_ex_noalloc(int(variant), ctypes.c_void_p(stream), ctypes.c_void_p(q_ptr),
                                      ctypes.c_void_p(k_ptr), ctypes.c_void_p(v_ptr), batch, heads, seq_len_q,
                                      seq_len_k, d_head, ctypes.byref(cfg), ctypes.byref(opts),
                                      ctypes.c_void_p(out_ptr)))


def release_stream_workspace(stream: int = 0) -> None:
    """Free the split workspace kept for `stream` (fa_release_stream_workspace)."""
    _check(lib().fa_release_stream_workspace(ctypes.c_void_p(stream)))


def describe_launch(variant: int, batch: int, heads: int, seq_len_q: int, seq_len_k: int, d_head: int,
                    causal: bool, path: int = PATH_AUTO, num_splits: int = 0, dtype: int = DTYPE_F32) -> str:
    """Kernel name(s) and grid a call would launch (launches nothing)."""
    opts = _COpts(0.0, int(path), int(num_splits), int(dtype))
    buf = ctypes.create_string_buffer(512)
    _check(lib().fa_describe_launch(int(variant), batch, heads, seq_len_q, seq_len_k, d_head,
                                    1 if causal else 0, ctypes.byref(opts), buf, len(buf)))
    return buf.value.decode()


PROBE_MFMA_F32_32X32X2 = 0
PROBE_MFMA_F32_16X16X4 = 1
PROBE_MFMA_BF16_16X16X32 = 2
PROBE_COPY = 3
PROBE_MFMA_BF16_32X32X16 = 4
PROBE_READ = 5


def probe_launch(kind: int, stream: int, buf: int, nbytes: int, iters: int = 0) -> float:
    """Queue one peak-probe kernel (fa_probe_launch) on `stream` over device
    memory `buf` (`nbytes` long); returns its work: FLOP for the MFMA probes,
    bytes read + written for the copy, bytes read for the read stream.  The
    caller times it."""
    if not 0 <= int(iters) < 1 << 32:
        raise FaError(FA_ERR_INVALID_ARG, "iters must fit 32 bits")
    work = ctypes.c_double(0.0)
    _check(lib().fa_probe_launch(int(kind), ctypes.c_void_p(stream), ctypes.c_void_p(buf), int(nbytes),
                                 int(iters), ctypes.byref(work)))
    return work.value


def init() -> None:
    """Load the gfx950 code object on the current device; raises without one."""
    _check(lib().fa_init())
